"""The C ABI: libh3mi.so loads without a GPU, exports every function that
include/h3mi.h declares, and rejects bad arguments before touching a device."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "h3mi.h")
LIB = os.path.join(ROOT, "minimax-h3-multi-dgx-spark_amd", "h3mi", "libh3mi.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(h3mi_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_abi():
    names = declared_functions()
    for must in ("h3mi_w8a8_gemm_bf16", "h3mi_w8a8_gemm_i32", "h3mi_quant_rowwise_i8", "h3mi_norm_mod_bf16",
                 "h3mi_gate_norm_mod_bf16", "h3mi_gate_bf16", "h3mi_last_error", "h3mi_w8a8_supported"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_the_abi():
    from h3mi import _lib
    assert set(_lib.SIGNATURES) == set(declared_functions())
    assert _lib.lib.h3mi_abi_version() == _lib.ABI_VERSION


def _err(status):
    from h3mi import _lib
    return status, _lib.lib.h3mi_last_error().decode()


P = ctypes.c_void_p


@pytest.mark.parametrize("M,N,K,ldx,ldw,ldo,code,msg", [
    (64, 64, 100, 100, 100, 64, 1, "multiple of 128"),
    (64, 66, 128, 128, 128, 66, 1, "multiple of 4"),
    (64, 64, 128, 120, 128, 64, 1, "leading dimension"),
    (64, 64, 128, 136, 128, 64, 2, "multiples of 16"),
    (64, 64, 128, 128, 128, 62, 1, "leading dimension"),
    (-1, 64, 128, 128, 128, 64, 1, "bad sizes"),
    # a 384-row tile's last row offset, 383 * ld, must fit in 32 bits (ld 2^22 + 16 passed the old 256-row bound)
    (64, 64, 128, (1 << 22) + 16, 128, 64, 1, "too large"),
    (64, 64, 128, 128, (1 << 22) + 16, 64, 1, "too large"),
])
def test_gemm_argument_errors(M, N, K, ldx, ldw, ldo, code, msg):
    from h3mi import _lib
    st, m = _err(_lib.lib.h3mi_w8a8_gemm_bf16(P(4096), P(8192), P(16384), P(32768), None, P(65536), M, N, K,
                                               ldx, ldw, ldo, None))
    assert st == code and msg in m


def test_gemm_alignment_and_alias_errors():
    from h3mi import _lib
    L = _lib.lib
    st, m = _err(L.h3mi_w8a8_gemm_bf16(P(4096 + 8), P(8192), P(16384), P(32768), None, P(1 << 20), 64, 64, 128,
                                        128, 128, 64, None))
    assert st == _lib.EALIGN
    st, m = _err(L.h3mi_w8a8_gemm_bf16(P(4096), P(1 << 20), P(16384), P(32768), None, P(4096), 64, 64, 128,
                                        128, 128, 64, None))
    assert st == _lib.EALIAS
    st, m = _err(L.h3mi_w8a8_gemm_i32(None, P(8192), P(1 << 20), 64, 64, 128, 128, 128, 64, None))
    assert st == _lib.EINVAL and "null" in m
    assert L.h3mi_w8a8_gemm_bf16(None, None, None, None, None, None, 0, 64, 128, 128, 128, 64, None) == 0


def test_quant_and_norm_argument_errors():
    from h3mi import _lib
    L = _lib.lib
    assert _err(L.h3mi_quant_rowwise_i8(P(4096), P(8192), P(12288), 4, 100, 100, None))[0] == _lib.EINVAL
    assert _err(L.h3mi_quant_rowwise_i8(P(4096), P(8192), P(12288), 4, 65536, 65536, None))[0] == _lib.EINVAL
    assert _err(L.h3mi_quant_rowwise_i8(P(4104), P(8192), P(12288), 4, 64, 64, None))[0] == _lib.EALIGN
    st, m = _err(L.h3mi_norm_mod_bf16(P(4096), P(8192), P(12288), P(16384), P(20480), P(1 << 20), 4, 66, 1,
                                      ctypes.c_float(1e-6), None))
    assert st == _lib.EINVAL and "multiple of 4" in m
    st, m = _err(L.h3mi_norm_mod_bf16_ex(P(4096), P(8192), P(12288), P(16384), P(20480), P(1 << 20), 4, 64, 1,
                                         ctypes.c_float(1e-6), 7, 0, None, None, None))
    assert st == _lib.EINVAL and "order" in m
    st, m = _err(L.h3mi_gate_norm_mod_bf16(P(4096), P(4096 + 64), P(1 << 20), P(8192), P(12288), P(16384),
                                           P(20480), P(1 << 21), 4, 64, 1, ctypes.c_float(1e-6), None))
    assert st == _lib.EALIAS and "o overlaps x" in m
    st, m = _err(L.h3mi_gate_bf16(P(4096), P(1 << 20), P(4096), P(8192), 4, 64, 1, None))
    assert st == _lib.EALIAS
    assert L.h3mi_gate_bf16(None, None, None, None, 0, 64, 1, None) == 0


def test_norm_register_limit_error():
    """Rows wider than the widest register-resident kernel are refused from the
    sizes alone: the pointers are null, so nothing could be launched."""
    from h3mi import _lib
    L = _lib.lib
    st, m = _err(L.h3mi_norm_mod_bf16(None, None, None, None, None, None, 1, 65536 + 4, 1, ctypes.c_float(1e-6), None))
    assert st == _lib.EINVAL and "register-resident limit" in m
    # the reference order (128 threads) has half the width
    st, m = _err(L.h3mi_norm_mod_bf16_ex(None, None, None, None, None, None, 1, 32768 + 4, 1, ctypes.c_float(1e-6),
                                         1, 0, None, None, None))
    assert st == _lib.EINVAL and "register-resident limit" in m


def test_config_registry():
    import h3mi
    names = h3mi.list_configs()
    assert len(names) == len(set(names)) >= 3
    from h3mi._lib import H3miError
    with pytest.raises(H3miError):
        h3mi.set_config("no-such-config")
    h3mi.set_config(names[-1])
    try:
        assert h3mi.config_for(4096, 4096, 4096) == names[-1]
    finally:
        h3mi.set_config("auto")
    assert h3mi.config_for(32768, 15360, 5120) != h3mi.config_for(256, 256, 256)


def test_norm_orders():
    import h3mi
    assert h3mi.order_info("ref") == (128, 4, 32)
    assert h3mi.order_info("default") == (256, 4, 64)


def test_fused_quant_argument_errors():
    """The norm + quantizer entry points reject shapes the fused kernel does
    not take and overlapping outputs, before any launch."""
    from h3mi import _lib
    L = _lib.lib
    f = ctypes.c_float(1e-6)
    # N % 8 != 0, N > 8192
    st, m = _err(L.h3mi_norm_mod_quant_i8(P(4096), P(8192), P(12288), P(16384), P(20480), None, P(1 << 20),
                                          P(1 << 21), 4, 68, 1, f, None))
    assert st == _lib.EINVAL and "multiple of 8" in m
    st, m = _err(L.h3mi_norm_mod_quant_i8(P(4096), P(8192), P(12288), P(16384), P(20480), None, P(1 << 24),
                                          P(1 << 25), 4, 8200, 1, f, None))
    assert st == _lib.EINVAL
    # q overlapping x
    st, m = _err(L.h3mi_norm_mod_quant_i8(P(1 << 20), P(8192), P(12288), P(16384), P(20480), None, P((1 << 20) + 64),
                                          P(1 << 22), 4, 64, 1, f, None))
    assert st == _lib.EALIAS and "q overlaps" in m
    # qs overlapping q
    st, m = _err(L.h3mi_gate_norm_mod_quant_i8(P(1 << 20), P(1 << 21), P(4096), P(8192), P(12288), P(16384),
                                               P(20480), None, P(1 << 22), P((1 << 22) + 16), 4, 64, 1, f, None))
    assert st == _lib.EALIAS and "qs overlaps" in m
    # null q
    st, m = _err(L.h3mi_norm_mod_quant_i8(P(4096), P(8192), P(12288), P(16384), P(20480), None, None, P(1 << 22),
                                          4, 64, 1, f, None))
    assert st == _lib.EINVAL and "null" in m
    assert L.h3mi_norm_mod_quant_i8(None, None, None, None, None, None, None, None, 0, 64, 1, f, None) == 0


def test_convrot_argument_errors():
    """The ConvRot quantizer rejects what its kernels do not take, before any launch."""
    from h3mi import _lib
    L = _lib.lib
    q, s = P(1 << 24), P(1 << 25)
    cases = [
        ((P(4096), q, s, 4, 1024, 1024, 128, 0), _lib.EINVAL, "group size"),
        ((P(4096), q, s, 4, 1024, 1024, 256, 2), _lib.EINVAL, "activation"),
        ((P(4096), q, s, 4, 1000, 1000, 256, 0), _lib.EINVAL, "multiple of 256"),
        ((P(4096), q, s, 4, 33024, 33024, 256, 0), _lib.EINVAL, "exceeds"),
        ((P(4096), q, s, 4, 1024, 1024, 256, 1), _lib.EALIGN, "ldx"),       # swiglu needs 2K columns
        ((P(4096), q, s, 4, 1024, 1028, 256, 0), _lib.EALIGN, "ldx"),
        ((P(4104), q, s, 4, 1024, 1024, 256, 0), _lib.EALIGN, "alignment"),
        ((P(4096), P((1 << 24) + 8), s, 4, 1024, 1024, 256, 0), _lib.EALIGN, "alignment"),
        ((P(1 << 24), P((1 << 24) + 4096), s, 4, 1024, 1024, 256, 0), _lib.EALIAS, "overlap"),
        ((None, q, s, 4, 1024, 1024, 256, 0), _lib.EINVAL, "null"),
        ((P(4096), q, s, -1, 1024, 1024, 256, 0), _lib.EINVAL, "bad sizes"),
    ]
    for args, code, msg in cases:
        st, m = _err(L.h3mi_quant_convrot_i8(*args, None))
        assert st == code and msg in m, (args, st, m)
    assert L.h3mi_quant_convrot_i8(None, None, None, 0, 1024, 1024, 256, 0, None) == 0


def test_rms_rope_argument_errors():
    """The q/k RMSNorm + RoPE entry rejects what its kernel does not take, and
    q / k views whose heads would overlap, before any launch."""
    from h3mi import _lib
    L = _lib.lib
    f = ctypes.c_float(1e-6)
    q, k, t, w = P(1 << 24), P(1 << 25), P(1 << 26), P(1 << 27)
    cases = [
        ((q, k, t, w, w, 4, 2, 96, 192, 192, 96), _lib.EINVAL, "head dim"),
        ((q, k, t, w, w, 4, 2, 128, 256, 256, 72), _lib.EINVAL, "multiple of 16"),
        ((q, k, t, w, w, 4, 2, 128, 256, 256, 256), _lib.EINVAL, "multiple of 16"),
        ((q, k, t, w, w, 4, 2, 128, 200, 256, 128), _lib.EALIGN, "token strides"),
        ((q, k, None, w, w, 4, 2, 128, 256, 256, 128), _lib.EINVAL, "null"),
        ((P((1 << 24) + 8), k, t, w, w, 4, 2, 128, 256, 256, 128), _lib.EALIGN, "alignment"),
        ((q, P((1 << 24) + 128), t, w, w, 4, 2, 128, 768, 768, 128), _lib.EALIAS, "heads overlap"),  # k 64 elements into q's heads
        ((q, P((1 << 24) + 512), t, w, w, 4, 2, 128, 768, 512, 128), _lib.EALIAS, "overlap"),
        ((q, k, P((1 << 24) + 64), w, w, 4, 2, 128, 256, 256, 128), _lib.EALIAS, "table"),
    ]
    for args, code, msg in cases:
        st, m = _err(L.h3mi_rms_rope_split_half_bf16(*args, f, 0, None, None))
        assert st == code and msg in m, (args, st, m)
    # q and k as the first two thirds of one qkv buffer [S, 3 * H * D] are accepted up to the launch
    assert L.h3mi_rms_rope_split_half_bf16(q, k, t, w, w, 0, 2, 128, 768, 768, 128, f, 0, None, None) == 0
    assert L.h3mi_rms_rope_split_half_bf16(q, P((1 << 24) + 512), None, w, w, 0, 2, 128, 768, 768, 0, f, 0, None, None) == 0


@pytest.mark.parametrize("M,N,K,tile", [
    (32768, 15360, 5120, "d_bm256_bn384_bk128_s2_g8_w8m_l4_a1_sw_res"),   # QKV
    (32768, 13824, 5120, "d_bm256_bn384_bk128_s2_g8_w8m_l4_a1_sw_res"),   # MLP up
    (32768, 5120, 13824, "d_bm256_bn320_bk128_s2_g4_w4x2_l4_sw_res"),     # MLP down: 8 whole rounds of 256x320
    (4096, 15360, 5120, "d_bm256_bn320_bk128_s2_g4_w4x2_l4_sw_res"),      # the shard: 3 whole rounds
    (19200, 21504, 5376, "d_bm256_bn384_bk128_s2_g8_w8m_l4_a1_sw_res"),   # H3 qkv
    (19200, 5376, 7168, "d_bm320_bn256_bk128_s2_g4_w8m_st1_sw_res"),      # H3 out: 4.92 rounds of 320x256
    (19200, 28672, 5376, "d_bm256_bn384_bk128_s2_g4_w8m_l4_a1_sw_res"),   # H3 fc1: operands past 240 MiB
    (38400, 21504, 5376, "d_bm256_bn384_bk128_s2_g4_w8m_l4_a1_sw_res"),   # H3 qkv at 38400 tokens
    (24576, 21504, 5376, "d_bm256_bn384_bk128_s2_g8_w8m_l4_a1_sw_res"),   # 236 MiB of operands: groups of 8
    (19200, 5376, 14336, "d_bm320_bn256_bk128_s2_g4_w8m_st1_sw_res"),     # H3 fc2
    (2048, 3072, 3072, "d_bm128_bn192_bk128_s2_g8_w2x2_sw_k2"),           # C0: one split-K tile per CU
    (512, 10240, 5120, "d_bm128_bn192_bk128_s2_g8_w2x2_sw_k2"),           # cross-attention KV projection
    (1024, 3072, 3072, "d_bm128_bn128_bk128_s2_g4_o2"),                   # 192 small tiles
    (1536, 4096, 4096, "d_bm128_bn128_bk128_s2_g4_o2"),                   # 264 split-K tiles: two rounds
    (2048, 3072, 3200, "d_bm128_bn128_bk128_s2_g4_o2"),                   # K % 256 != 0: no split-K
])
def test_heuristic_picks_the_measured_tiling(M, N, K, tile):
    """The tiling the heuristic picks at the workload shapes, each the winner of a same-process A/B on the box
    (the library assumes MI355X's 256 CUs when no GPU is visible, as here)."""
    import h3mi
    assert h3mi.config_for(M, N, K) == tile


def test_buffer_probe_argument_errors():
    """The range-check probe rejects its arguments before any launch."""
    from h3mi import _lib
    L = _lib.lib
    cases = [
        ((None, 4096, P(8192), 0, 0, P(16384)), _lib.EINVAL, "null"),
        ((P(4096), -1, P(8192), 0, 0, P(16384)), _lib.EINVAL, "records"),
        ((P(4096), 1 << 31, P(8192), 0, 0, P(16384)), _lib.EINVAL, "records"),
        ((P(4096), 4096, P(8192), -16, 0, P(16384)), _lib.EINVAL, "soffset"),
        ((P(4096), 4096, P(8192), 0, 512, P(16384)), _lib.EINVAL, "ioffset"),
        ((P(4096), 4096, P(8192), 0, 0, P(16392)), _lib.EALIGN, "aligned"),
    ]
    for args, code, msg in cases:
        st, m = _err(L.h3mi_debug_buffer_lds_load(*args, None))
        assert st == code and msg in m, (args, st, m)
