"""Device primitives the kernels are built from, pinned in isolation:
fp32 -> bf16 rounding (the gfx950 hardware convert), the two rsqrt modes, and
the buffer range check of the GEMM's LDS-DMA operand loads."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _lib():
    from h3mi import _lib
    return _lib


def _dev_bf16(f32):
    L = _lib()
    x = torch.from_numpy(np.ascontiguousarray(f32, np.float32)).cuda()
    out = torch.empty(x.numel(), dtype=torch.int16, device="cuda")
    L.check(L.lib.h3mi_debug_bf16_rne(L.ptr(x), L.ptr(out), x.numel(), L.stream_of(x)))
    return out.cpu().numpy().view(np.uint16)


def _dev_rsqrt(f32, mode):
    L = _lib()
    x = torch.from_numpy(np.ascontiguousarray(f32, np.float32)).cuda()
    out = torch.empty_like(x)
    L.check(L.lib.h3mi_debug_rsqrt_f32(L.ptr(x), L.ptr(out), x.numel(), mode, L.stream_of(x)))
    return out.cpu().numpy()


def test_bf16_convert_matches_integer_rne_on_all_high_halves():
    # every sign/exponent/top-7-mantissa pattern x low halves that straddle
    # the rounding boundary (0x7FFF, 0x8000 tie, 0x8001) and random ones
    hi = np.arange(65536, dtype=np.uint32) << 16
    lows = [0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x4000, 0xC000]
    g = np.random.default_rng(0)
    pats = np.concatenate([hi | lo for lo in lows] + [hi | g.integers(0, 65536, 65536).astype(np.uint32)])
    f = pats.view(np.float32)
    finite = np.isfinite(f)
    got = _dev_bf16(f[finite])
    ref = O.f32_to_bf16_bits(f[finite])
    assert np.array_equal(got, ref)


def test_rsqrt_rn_mode_matches_oracle():
    g = np.random.default_rng(1)
    v = np.concatenate([np.float32(10.0) ** g.uniform(-37, 37, 200_000).astype(np.float32),
                        (g.random(100_000) * 4 + 1e-6).astype(np.float32)]).astype(np.float32)
    got = _dev_rsqrt(v, 1)
    ref = np.array([O.rsqrt_rn(x) for x in v[:20000]], np.float32)
    assert np.array_equal(got[:20000].view(np.uint32), ref.view(np.uint32))
    # the rest against an independent fp64 reference: within 0.5 ulp + tiny
    r64 = 1.0 / np.sqrt(v.astype(np.float64))
    ulp = np.spacing(got.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - r64) <= 0.5 * ulp * (1 + 1e-9))


def test_rsqrt_hw_mode_within_one_ulp():
    g = np.random.default_rng(2)
    v = (np.float32(10.0) ** g.uniform(-30, 30, 100_000)).astype(np.float32)
    hw = _dev_rsqrt(v, 0)
    rn = _dev_rsqrt(v, 1)
    d = np.abs(hw.view(np.int32).astype(np.int64) - rn.view(np.int32).astype(np.int64))
    assert d.max() <= 1


def _dev_lds_load(buf, records, voff, soffset, ioffset):
    L = _lib()
    v = torch.tensor(voff, dtype=torch.int32, device="cuda")
    out = torch.zeros(1024, dtype=torch.uint8, device="cuda")
    L.check(L.lib.h3mi_debug_buffer_lds_load(L.ptr(buf), records, L.ptr(v), soffset, ioffset, L.ptr(out),
                                             L.stream_of(buf)))
    return out.cpu().numpy().reshape(64, 16)


@pytest.mark.parametrize("records,lane_step,vbase,soffset,ioffset,n_in", [
    (8192, 16, 0, 8192 - 512, 0, 32),        # voffset < R and soffset < R, their sum >= R from lane 32
    (3584, 16, 0, 0, 3072, 32),              # voffset < R and instruction offset < R, sum >= R from lane 32
    (5632, 16, 0, 2048, 3072, 32),           # all three below R, the sum >= R from lane 32
    (6144, 16, 0, 2048, 3072, 64),           # all in range
    (8192, 16, 8192 - 1024, 0, 0, 64),       # voffset alone, up to the last byte
    (8192, 16, 8192 - 256, 0, 0, 16),        # voffset alone past R from lane 16
    (8192, 16, 0, 8192, 0, 0),               # soffset alone at R
    (8192, 16, 0, 2048, 1024, 64),
])
def test_lds_dma_range_check_covers_the_offset_sum(records, lane_step, vbase, soffset, ioffset, n_in):
    """The GEMM's operand loads put part of a row offset in soffset and part in
    the instruction offset (csrc/gemm_w8a8.hip, PAR loads) and rely on rows
    past M or N reading nothing.  A raw-buffer LDS-DMA load returns memory only
    when voffset + soffset + instruction offset + 16 <= records: lanes past
    that get no buffer bytes (zero, or the LDS left as it was), also where
    each offset alone is in range.  The buffer extends past `records` with a
    pattern that is never 0x00 or 0xAB, so a load that ignored part of the sum
    would return it (and would stay inside the allocation)."""
    span = vbase + lane_step * 63 + soffset + ioffset + 16
    n = max(span, records) + 4096
    pattern = (1 + (np.arange(n) % 127)).astype(np.uint8)
    buf = torch.from_numpy(pattern).cuda()
    voff = [vbase + lane_step * l for l in range(64)]
    got = _dev_lds_load(buf, records, voff, soffset, ioffset)
    for lane in range(64):
        a = voff[lane] + soffset + ioffset
        if a + 16 <= records:
            assert lane < n_in and np.array_equal(got[lane], pattern[a:a + 16]), lane
        else:
            assert lane >= n_in, lane
            assert np.all(got[lane] == 0) or np.all(got[lane] == 0xAB), (lane, got[lane])
