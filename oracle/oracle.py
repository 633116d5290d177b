"""numpy binding of liboracle.so (test infrastructure only; see oracle.c for what each function restates)."""
import ctypes
import os
import subprocess

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "liboracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _DIR], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i32, i64 = ctypes.c_int32, ctypes.c_int64
        L.oracle_attention_f64.restype = ctypes.c_int
        L.oracle_attention_f64.argtypes = [i32, i32, i32, i32, i32, i32, i32, ctypes.c_double, P, i64, P, P, i64,
                                           P, i64, P]
        L.oracle_cpu_attend_f32.restype = ctypes.c_int
        L.oracle_cpu_attend_f32.argtypes = [i32, i32, i32, i32, i32, i32, i32, ctypes.c_float, P, i64, P, P, i64,
                                            P, i64, i32]
        L.oracle_f16_to_f32.restype = None
        L.oracle_f16_to_f32.argtypes = [P, P, i64]
        L.oracle_f32_to_f16.restype = None
        L.oracle_f32_to_f16.argtypes = [P, P, i64]
        L.oracle_linear_f64.restype = ctypes.c_int
        L.oracle_linear_f64.argtypes = [i32, i32, i32, ctypes.c_uint32, i32, ctypes.c_float, P, i64, P, P, P, P]
        L.oracle_rope_f32.restype = None
        L.oracle_rope_f32.argtypes = [i32, ctypes.c_float, i32, i32, P, P, i64]
        _lib = L
    return _lib


def _f16(a):
    a = np.ascontiguousarray(a)
    if a.dtype != np.float16 or a.ndim != 2:
        raise ValueError("expected a 2-D float16 array")
    return a


def attention_f64(q, k, v, n_head, n_head_kv, head_dim, scale, p0=0, causal=True, n_kv=None):
    """Brute-force f64 attention of query rows q [n_q][..] over caches k/v [n_kv][..] (float16 arrays).
    Returns (out [n_q][n_head*hd] f64, lse [n_q][n_head] f64)."""
    q, k, v = _f16(q), _f16(k), _f16(v)
    n_q = q.shape[0]
    n_kv = k.shape[0] if n_kv is None else n_kv
    out = np.zeros((n_q, n_head * head_dim), np.float64)
    lse = np.zeros((n_q, n_head), np.float64)
    rc = lib().oracle_attention_f64(n_head, n_head_kv, head_dim, n_q, p0, n_kv, 1 if causal else 0, float(scale),
                                    q.ctypes.data, q.shape[1], k.ctypes.data, v.ctypes.data, k.shape[1],
                                    out.ctypes.data, out.shape[1], lse.ctypes.data)
    if rc:
        raise ValueError(f"oracle_attention_f64 rejected the arguments ({rc})")
    return out, lse


def cpu_attend_f32(q, k, v, n_head, n_head_kv, head_dim, scale, p0=0, causal=True, n_kv=None, n_threads=1):
    """The restated reference CPU attention on float32 arrays (convert f16 with astype outside any timing)."""
    q, k, v = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v))
    n_q = q.shape[0]
    n_kv = k.shape[0] if n_kv is None else n_kv
    out = np.zeros((n_q, n_head * head_dim), np.float32)
    rc = lib().oracle_cpu_attend_f32(n_head, n_head_kv, head_dim, n_q, p0, n_kv, 1 if causal else 0, float(scale),
                                     q.ctypes.data, q.shape[1], k.ctypes.data, v.ctypes.data, k.shape[1],
                                     out.ctypes.data, out.shape[1], n_threads)
    if rc:
        raise ValueError(f"oracle_cpu_attend_f32 failed ({rc})")
    return out


def f16_to_f32(a):
    """Exact binary16 -> binary32 conversion by the oracle's own routine (checked against numpy's)."""
    a = np.ascontiguousarray(a, dtype=np.float16)
    out = np.empty(a.shape, np.float32)
    lib().oracle_f16_to_f32(a.ctypes.data, out.ctypes.data, a.size)
    return out


def rope_f32(x, mode, base, head_dim, pos):
    """oracle_rope_f32 on an f32 array whose last axis holds whole heads (size a multiple of head_dim)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().oracle_rope_f32(mode, base, head_dim, pos, x.ctypes.data, y.ctypes.data, x.size // head_dim)
    return y


def f32_to_f16(a):
    """Round-to-nearest-even binary32 -> binary16 (oracle_f32_to_f16), as float16 array."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16(a.ctypes.data, out.ctypes.data, a.size)
    return out.view(np.float16)


def linear_f64(x, w, flags=0, half_input=False, eps=1e-5, gamma=None, bias=None, y0=None):
    """oracle_linear_f64: x f32 [M][>=K], w f16 [N][K]; returns Y float64 [M][N] (y0: the accumulate input)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float16)
    M, N, K = x.shape[0], w.shape[0], w.shape[1]
    y = np.zeros((M, N)) if y0 is None else np.array(y0, dtype=np.float64, order="C")
    g = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = lib().oracle_linear_f64(M, N, K, flags, 1 if half_input else 0, eps, x.ctypes.data, x.shape[1],
                                 w.ctypes.data, None if g is None else g.ctypes.data,
                                 None if b is None else b.ctypes.data, y.ctypes.data)
    if rc:
        raise ValueError(f"oracle_linear_f64 failed ({rc})")
    return y


def self_attention_f64(qkv, heads, scale):
    """The IR SelfAttention op in f64 on packed rows qkv [B][N][3E] (any float dtype; f16 is exact in f64): per batch
    element and head softmax(scale q k^T) v without a mask -- the reference's test oracle attention_ref
    (tests/unit/test_backend_ggml.cpp:650-675): scores in double, max subtracted, exponentials normalized by their sum.
    Returns y [B][N][E] f64."""
    qkv = np.asarray(qkv)
    B, N, E3 = qkv.shape
    E = E3 // 3
    hd = E // heads
    y = np.zeros((B, N, E), np.float64)
    for b in range(B):
        x = qkv[b].astype(np.float64)
        for h in range(heads):
            q = x[:, h * hd:(h + 1) * hd]
            k = x[:, E + h * hd:E + (h + 1) * hd]
            v = x[:, 2 * E + h * hd:2 * E + (h + 1) * hd]
            s = scale * (q @ k.T)
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            y[b, :, h * hd:(h + 1) * hd] = (p / p.sum(axis=1, keepdims=True)) @ v
    return y
