"""numpy front end of the CPU oracle (oracle/h3_oracle.c).

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module, and only to check or time against the
product; the product library never calls it.

Arrays are numpy; bf16 tensors travel as uint16 bit patterns.  Each wrapper
names the reference function it restates (paths relative to the reference
repository root; LF = comfyui_nodes/h3-linear-fast, FG = comfyui_nodes/h3-fuse-graph).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "libh3oracle.so")

# Reduction order of the reference's fused norms (FG/h3_fuse_kernels.py:42-43):
# 128 logical threads, 4-element chunks, 32-lane shuffle tree.
REF_ORDER = (128, 4, 32)


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    if not os.path.exists(_SO):
        build()
    lib = ctypes.CDLL(_SO)
    P = ctypes.c_void_p
    I = ctypes.c_int64
    F = ctypes.c_float
    C = ctypes.c_int
    lib.h3o_rbf16.argtypes = [F]
    lib.h3o_rbf16.restype = F
    lib.h3o_bf16_bits.argtypes = [F]
    lib.h3o_bf16_bits.restype = ctypes.c_uint16
    lib.h3o_rsqrt_rn.argtypes = [F]
    lib.h3o_rsqrt_rn.restype = F
    lib.h3o_quant_rowwise.argtypes = [P, I, I, I, P, P]
    lib.h3o_gemm_i32.argtypes = [P, P, I, I, I, I, I, P, I]
    lib.h3o_epilogue_bf16.argtypes = [P, I, P, P, P, I, I, P, I]
    lib.h3o_row_sumsq.argtypes = [P, I, C, C, C]
    lib.h3o_row_sumsq.restype = F
    lib.h3o_norm_mod.argtypes = [P, P, P, P, P, P, I, I, F, C, C, C, P, P, P]
    lib.h3o_gate_norm_mod.argtypes = [P, P, P, P, P, P, P, P, I, I, F, C, C, C, P, P, P]
    lib.h3o_gate.argtypes = [P, P, P, P, I, I]
    lib.h3o_exp_neg.argtypes = [F]
    lib.h3o_exp_neg.restype = F
    lib.h3o_silu.argtypes = [F]
    lib.h3o_silu.restype = F
    lib.h3o_rcp12.argtypes = [F]
    lib.h3o_rcp12.restype = F
    lib.h3o_fwht256.argtypes = [P]
    lib.h3o_convrot_quant.argtypes = [P, I, I, I, C, P, P]
    lib.h3o_rms_rope_split_half.argtypes = [P, P, P, I, I, I, I, I, F, C, C, C, P, P]
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ----------------------------------------------------------------------------- bf16

def f32_to_bf16_bits(a):
    """Vectorised RNE fp32 -> bf16 bits (same rule as h3o_bf16_bits, NaN kept quiet)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_bits_to_f32(b):
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rbf16(v):
    """FG/h3_fuse_kernels.py:78-85 on one fp32 value."""
    return lib().h3o_rbf16(float(v))


def rsqrt_rn(v):
    """Correctly rounded fp32 1/sqrt(v)."""
    return lib().h3o_rsqrt_rn(float(v))


# ----------------------------------------------------------------------------- W8A8

def quant_rowwise(x_bits):
    """Per-token int8 quantizer (replaces LF/h3_linear_fast_patch.py:90-95's
    external quantizer; semantics: s = absmax/127, q = clamp(rne(x/s), +-127))."""
    x = _c(x_bits, np.uint16)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    lib().h3o_quant_rowwise(_p(x), M, K, K, _p(q), _p(s))
    return q, s


def gemm_i32(xq, w):
    """LF/int8_gemm_triton.py:47-60: acc[m,n] = sum_k xq[m,k]*w[n,k]."""
    xq = _c(xq, np.int8)
    w = _c(w, np.int8)
    M, K = xq.shape
    N = w.shape[0]
    assert w.shape[1] == K
    acc = np.empty((M, N), np.int32)
    lib().h3o_gemm_i32(_p(xq), _p(w), M, N, K, K, K, _p(acc), N)
    return acc


def epilogue_bf16(acc, xs, ws, bias_bits=None):
    """LF/int8_gemm_triton.py:61-66: bf16((f32(acc)*xs[m])*ws[n]) (+ bias)."""
    acc = _c(acc, np.int32)
    M, N = acc.shape
    xs = _c(np.reshape(xs, (M,)), np.float32)
    ws = _c(np.reshape(ws, (N,)), np.float32)
    b = None if bias_bits is None else _c(bias_bits, np.uint16)
    out = np.empty((M, N), np.uint16)
    lib().h3o_epilogue_bf16(_p(acc), N, _p(xs), _p(ws), _p(b), M, N, _p(out), N)
    return out


def w8a8_linear(x_bits, w, ws, bias_bits=None):
    """Quantize, int32 GEMM, epilogue: the whole W8A8 linear in oracle arithmetic."""
    q, s = quant_rowwise(x_bits)
    acc = gemm_i32(q, w)
    return epilogue_bf16(acc, s, ws, bias_bits), q, s, acc


# ----------------------------------------------------------------------------- fused norms

def row_sumsq(xrow_f32, order=REF_ORDER):
    x = _c(xrow_f32, np.float32)
    numx, vec, ws = order
    return lib().h3o_row_sumsq(_p(x), x.shape[0], numx, vec, ws)


def norm_mod(x_bits, w_bits, eps, ridx, s1_bits, sh_bits, order=REF_ORDER, rstd=None):
    """FG/h3_fuse_kernels.py:88-114.  rstd=None: correctly rounded rsqrt;
    else the per-row rstd to use.  Returns (h, var, rstd_used)."""
    x = _c(x_bits, np.uint16)
    S, N = x.shape
    h = np.empty((S, N), np.uint16)
    var = np.empty((S,), np.float32)
    rs = np.empty((S,), np.float32)
    rin = None if rstd is None else _c(rstd, np.float32)
    numx, vec, wsz = order
    lib().h3o_norm_mod(_p(x), _p(_c(w_bits, np.uint16)), _p(_c(ridx, np.int32)),
                       _p(_c(s1_bits, np.uint16)), _p(_c(sh_bits, np.uint16)), _p(h),
                       S, N, float(eps), numx, vec, wsz, _p(rin), _p(var), _p(rs))
    return h, var, rs


def gate_norm_mod(x_bits, o_bits, g_bits, w_bits, eps, ridx, s1_bits, sh_bits,
                  order=REF_ORDER, rstd=None):
    """FG/h3_fuse_kernels.py:117-155.  Returns (x_new, h, var, rstd_used); the
    input array is not modified."""
    x = np.array(x_bits, dtype=np.uint16, copy=True, order="C")
    S, N = x.shape
    h = np.empty((S, N), np.uint16)
    var = np.empty((S,), np.float32)
    rs = np.empty((S,), np.float32)
    rin = None if rstd is None else _c(rstd, np.float32)
    numx, vec, wsz = order
    lib().h3o_gate_norm_mod(_p(x), _p(_c(o_bits, np.uint16)), _p(_c(g_bits, np.uint16)),
                            _p(_c(w_bits, np.uint16)), _p(_c(ridx, np.int32)),
                            _p(_c(s1_bits, np.uint16)), _p(_c(sh_bits, np.uint16)), _p(h),
                            S, N, float(eps), numx, vec, wsz, _p(rin), _p(var), _p(rs))
    return x, h, var, rs


def gate(x_bits, o_bits, g_bits, ridx):
    """FG/h3_fuse_kernels.py:158-167.  Returns the new x (input untouched)."""
    x = np.array(x_bits, dtype=np.uint16, copy=True, order="C")
    S, N = x.shape
    lib().h3o_gate(_p(x), _p(_c(o_bits, np.uint16)), _p(_c(g_bits, np.uint16)),
                   _p(_c(ridx, np.int32)), S, N)
    return x


# ----------------------------------------------------------------------------- ConvRot quantizer

ACTS = {None: 0, "none": 0, "swiglu": 1}


def exp_neg(x):
    """e^x for x <= 0 (argument clamped at -86) by the stated Cody-Waite + Taylor method."""
    f = lib().h3o_exp_neg
    return np.array([f(float(v)) for v in np.ravel(np.asarray(x, np.float32))], np.float32).reshape(np.shape(x))


def rcp12(d):
    """1/d on [1, 2]: linear seed and three Newton steps."""
    f = lib().h3o_rcp12
    return np.array([f(float(v)) for v in np.ravel(np.asarray(d, np.float32))], np.float32).reshape(np.shape(d))


def silu(a):
    f = lib().h3o_silu
    return np.array([f(float(v)) for v in np.ravel(np.asarray(a, np.float32))], np.float32).reshape(np.shape(a))


def fwht256(v):
    """Unnormalised 256-point fast Walsh-Hadamard transform, stages 1..128 (returns a copy)."""
    y = np.array(v, dtype=np.float32, copy=True, order="C")
    assert y.shape == (256,)
    lib().h3o_fwht256(_p(y))
    return y


def convrot_quant(x_bits, act=None):
    """ConvRot quantizer standing in for comfy-kitchen's
    _C.quantize_int8_rowwise_convrot64 (called at LF/h3_linear_fast_patch.py:90-95,
    tests/bench_linear.py:33-40): 256-group Hadamard rotation /16, then per-row
    int8.  PARITY UNPINNED against the reference (comfy-kitchen is not vendored);
    pinned to the mathematics in tests/test_oracle_pins.py.  x bf16 bits [M, K]
    or [M, 2K] for act="swiglu" -> (q int8 [M, K], s fp32 [M])."""
    x = _c(x_bits, np.uint16)
    M, Kin = x.shape
    a = ACTS[act]
    K = Kin // 2 if a == 1 else Kin
    assert K % 256 == 0 and (a == 0 or Kin == 2 * K)
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    lib().h3o_convrot_quant(_p(x), M, K, Kin, a, _p(q), _p(s))
    return q, s


# ----------------------------------------------------------------------------- q/k RMSNorm + RoPE

def rms_rope_split_half(x_bits, tab_bits, w_bits, eps, rot, order=(256, 4, 64), rstd=None):
    """RMSNorm of each (token, head) row then split-half RoPE, standing in for
    comfy-kitchen's ck.rms_rope_split_half_ as called at
    comfyui_nodes/minimax-h3-sp/minimax_sp/sp_forward.py:279-296.  PARITY
    UNPINNED against the reference (comfy-kitchen is not vendored); the
    definition (h3o_rms_rope_split_half) is the eager F.rms_norm -> RoPE
    sequence.  x bf16 bits [S, H, D]; tab bf16 bits [S, rot/2, 2, 2]; w [D];
    rstd: per-row rstd [S, H] to use (else the correctly rounded rsqrt).
    Returns (out, rstd_used); the input is not modified."""
    x = np.array(x_bits, dtype=np.uint16, copy=True, order="C")
    S, H, D = x.shape
    t = _c(tab_bits, np.uint16) if rot else np.zeros((1,), np.uint16)
    rs = np.empty((S, H), np.float32)
    rin = None if rstd is None else _c(rstd, np.float32)
    numx, vec, wsz = order
    lib().h3o_rms_rope_split_half(_p(x), _p(t), _p(_c(w_bits, np.uint16)), S, H, D, H * D, rot, float(eps),
                                  numx, vec, wsz, _p(rin), _p(rs))
    return x, rs
