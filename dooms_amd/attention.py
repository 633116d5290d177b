"""torch-tensor front end of the C ABI (plumbing: torch only supplies device memory and the stream).

Every call goes through libmx_attn.so; there is no CPU or PyTorch fallback. Tensors must be CUDA (HIP) float16 with a
unit stride along the feature dimension; row strides are taken from the tensors.
"""
import contextlib
import math

import torch

from . import _lib

# Tuning that calls without their own `tuning=` argument pass in their descriptors (see tuning()); None: the library's
# plans.
_default_tuning = None


@contextlib.contextmanager
def tuning(**fields):
    """Within the block, calls that do not pass `tuning=` use an mx_attn_tuning with these fields (decode_splits,
    decode_waves, decode_max_workgroups, prefill_plan); the library's plan for the others."""
    global _default_tuning
    saved = _default_tuning
    _default_tuning = dict(fields)
    try:
        yield
    finally:
        _default_tuning = saved


def _tuning(t):
    return _default_tuning if t is None else t


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _rows(t: torch.Tensor, name: str, dtype=torch.float16) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be 2-D [rows][features] with unit feature stride")
    return t


def prefill(q, k_cache, v_cache, *, n_head, n_head_kv, head_dim, p0=0, causal=True, n_kv=None, scale=None,
            out=None, lse=None, want_lse=False, workspace=None, tuning=None):
    """mx_attn_prefill: q [n_q][>= n_head*hd], caches [n_kv][>= n_head_kv*hd]. Returns (out, lse or None).
    workspace: "auto" (sized and zeroed here) or a zeroed uint8 device tensor runs mx_attn_prefill_ws, which takes the
    split-KV kernel for chunks of few rows; None runs mx_attn_prefill."""
    _rows(q, "q"), _rows(k_cache, "k_cache"), _rows(v_cache, "v_cache")
    if k_cache.stride(0) != v_cache.stride(0):
        raise ValueError("k_cache and v_cache must share a row stride")
    n_q = q.shape[0]
    if out is None:
        out = torch.empty(n_q, n_head * head_dim, dtype=torch.float16, device=q.device)
    _rows(out, "out")
    if want_lse and lse is None:
        lse = torch.empty(n_q, n_head, dtype=torch.float32, device=q.device)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    d = _lib.make_desc(n_head, n_head_kv, head_dim, n_q, q.stride(0), k_cache.stride(0), out.stride(0), scale,
                       p0=p0, n_kv=0 if n_kv is None else n_kv, causal=1 if causal else 0, tuning=_tuning(tuning))
    if workspace is None:
        _lib.check(_lib.prefill_raw(d, q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(),
                                    lse.data_ptr() if lse is not None else 0, _stream()))
        return out, lse
    if isinstance(workspace, str):
        workspace = new_workspace(_lib.prefill_workspace_bytes(d), q.device)
    _lib.check(_lib.prefill_ws_raw(d, q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(),
                                   lse.data_ptr() if lse is not None else 0, workspace.data_ptr(), workspace.numel(),
                                   _stream()))
    return out, lse


def decode_workspace_bytes(*, n_head, n_head_kv, head_dim, n_q, batch, max_kv_len, causal=False) -> int:
    d = _lib.make_desc(n_head, n_head_kv, head_dim, n_q, n_head * head_dim, n_head_kv * head_dim,
                       n_head * head_dim, 1.0, causal=1 if causal else 0)
    return _lib.decode_workspace_bytes(d, batch, max_kv_len)


def new_workspace(nbytes: int, device) -> torch.Tensor:
    """A decode workspace of nbytes (torch's caching allocator aligns it to 512 bytes), zeroed by the library."""
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
    _lib.check(_lib.decode_workspace_init(ws.data_ptr(), ws.numel(), _stream()))
    return ws


def decode(q, k_caches, v_caches, kv_len, *, n_head, n_head_kv, head_dim, n_q=1, causal=False, scale=None,
           out=None, lse=None, want_lse=False, workspace=None, tuning=None):
    """mx_attn_decode (float16 q) or mx_attn_decode_f32 (float32 q and output): q [batch*n_q][>= n_head*hd];
    k_caches/v_caches lists of [>= kv_len[b]][>= n_head_kv*hd] float16 tensors (entries may repeat); kv_len list of
    ints. Returns (out, lse or None)."""
    batch = len(kv_len)
    if len(k_caches) != batch or len(v_caches) != batch:
        raise ValueError("k_caches, v_caches and kv_len must have one entry per sequence")
    f32 = q.dtype == torch.float32
    _rows(q, "q", q.dtype if f32 else torch.float16)
    kv_stride = k_caches[0].stride(0)
    for t in list(k_caches) + list(v_caches):
        _rows(t, "cache")
        if t.stride(0) != kv_stride:
            raise ValueError("every cache must share one row stride")
    if out is None:
        out = torch.empty(q.shape[0], n_head * head_dim, dtype=q.dtype, device=q.device)
    _rows(out, "out", q.dtype)
    if want_lse and lse is None:
        lse = torch.empty(q.shape[0], n_head, dtype=torch.float32, device=q.device)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    d = _lib.make_desc(n_head, n_head_kv, head_dim, n_q, q.stride(0), kv_stride, out.stride(0), scale,
                       causal=1 if causal else 0, tuning=_tuning(tuning))
    if workspace is None:
        workspace = new_workspace(_lib.decode_workspace_bytes(d, batch, max(kv_len)), q.device)
    _lib.check((_lib.decode_f32_raw if f32 else _lib.decode_raw)(d, list(kv_len), q.data_ptr(), [t.data_ptr() for t in k_caches],
                               [t.data_ptr() for t in v_caches], out.data_ptr(),
                               lse.data_ptr() if lse is not None else 0, workspace.data_ptr(), workspace.numel(),
                               _stream()))
    return out, lse


def decode_rope(qkv, k_caches, v_caches, kv_len, *, n_head, n_head_kv, head_dim, rope_mode, rope_base=10000.0,
                scale=None, out=None, lse=None, want_lse=False, workspace=None, tuning=None):
    """mx_attn_decode_rope, the fused decode step: qkv f32 [batch][>= (n_head + 2 n_head_kv) hd] holds each sequence's
    new token unrotated (q | k | v); the token goes to position kv_len[b] - 1 of k_caches[b] / v_caches[b] (f16,
    written in place). Returns (out f32 [batch][n_head hd], lse or None)."""
    batch = len(kv_len)
    if len(k_caches) != batch or len(v_caches) != batch:
        raise ValueError("k_caches, v_caches and kv_len must have one entry per sequence")
    _rows(qkv, "qkv", torch.float32)
    kv_stride = k_caches[0].stride(0)
    for t in list(k_caches) + list(v_caches):
        _rows(t, "cache")
        if t.stride(0) != kv_stride:
            raise ValueError("every cache must share one row stride")
    if out is None:
        out = torch.empty(batch, n_head * head_dim, dtype=torch.float32, device=qkv.device)
    _rows(out, "out", torch.float32)
    if want_lse and lse is None:
        lse = torch.empty(batch, n_head, dtype=torch.float32, device=qkv.device)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    d = _lib.make_desc(n_head, n_head_kv, head_dim, 1, qkv.stride(0), kv_stride, out.stride(0), scale, causal=0,
                       tuning=_tuning(tuning))
    if workspace is None:
        workspace = new_workspace(_lib.decode_workspace_bytes(d, batch, max(kv_len)), qkv.device)
    _lib.check(_lib.decode_rope_raw(d, rope_mode, rope_base, list(kv_len), qkv.data_ptr(),
                                    [t.data_ptr() for t in k_caches], [t.data_ptr() for t in v_caches],
                                    out.data_ptr(), lse.data_ptr() if lse is not None else 0, workspace.data_ptr(),
                                    workspace.numel(), _stream()))
    return out, lse


def prefill_rope(qkv, k_cache, v_cache, *, n_head, n_head_kv, head_dim, rope_mode, rope_base=10000.0, p0=0,
                 causal=True, n_kv=None, scale=None, out=None, lse=None, want_lse=False, workspace=None,
                 tuning=None):
    """mx_attn_prefill_rope: qkv f32 [n_q][>= (n_head + 2 n_head_kv) hd] unrotated rows at positions p0 ..; their keys
    and values are written (rotated, f16) into rows p0 .. of k_cache / v_cache, then the chunk attends.
    Returns (out f32 [n_q][n_head hd], lse or None). workspace ("auto" or a zeroed uint8 device tensor) runs
    mx_attn_prefill_rope_ws."""
    _rows(qkv, "qkv", torch.float32), _rows(k_cache, "k_cache"), _rows(v_cache, "v_cache")
    if k_cache.stride(0) != v_cache.stride(0):
        raise ValueError("k_cache and v_cache must share a row stride")
    n_q = qkv.shape[0]
    if out is None:
        out = torch.empty(n_q, n_head * head_dim, dtype=torch.float32, device=qkv.device)
    _rows(out, "out", torch.float32)
    if want_lse and lse is None:
        lse = torch.empty(n_q, n_head, dtype=torch.float32, device=qkv.device)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    d = _lib.make_desc(n_head, n_head_kv, head_dim, n_q, qkv.stride(0), k_cache.stride(0), out.stride(0), scale,
                       p0=p0, n_kv=0 if n_kv is None else n_kv, causal=1 if causal else 0, tuning=_tuning(tuning))
    if workspace is None:
        _lib.check(_lib.prefill_rope_raw(d, rope_mode, rope_base, qkv.data_ptr(), k_cache.data_ptr(),
                                         v_cache.data_ptr(), out.data_ptr(), lse.data_ptr() if lse is not None else 0,
                                         _stream()))
        return out, lse
    if isinstance(workspace, str):
        workspace = new_workspace(_lib.prefill_workspace_bytes(d), qkv.device)
    _lib.check(_lib.prefill_rope_ws_raw(d, rope_mode, rope_base, qkv.data_ptr(), k_cache.data_ptr(),
                                        v_cache.data_ptr(), out.data_ptr(), lse.data_ptr() if lse is not None else 0,
                                        workspace.data_ptr(), workspace.numel(), _stream()))
    return out, lse


def linear(x, weights, *, out=None, gamma=None, bias=None, eps=1e-5, accumulate=False, out_f16=False):
    """mx_linear: x f32 [M][>= K]; weights: one f16 [N][K] tensor or a list of them (same shape, one launch);
    out: matching output tensor(s) (f32, or f16 with out_f16), created if None; gamma f32 [K] turns on the RMS norm;
    bias: f32 [N] tensor or list (None entries allowed). Returns the output tensor or list."""
    single = isinstance(weights, torch.Tensor)
    ws_list = [weights] if single else list(weights)
    _rows(x, "x", torch.float32)
    N, K = ws_list[0].shape
    for w in ws_list:
        _rows(w, "weight")
        if tuple(w.shape) != (N, K) or w.stride(0) != K:
            raise ValueError("weights must be contiguous [N][K] tensors of one shape")
    odt = torch.float16 if out_f16 else torch.float32
    if out is None:
        outs = [torch.empty(x.shape[0], N, dtype=odt, device=x.device) for _ in ws_list]
    else:
        outs = [out] if single else list(out)
    for o in outs:
        _rows(o, "out", odt)
    if len({o.stride(0) for o in outs}) != 1:
        raise ValueError("outputs must share one row stride")
    bl = None
    if bias is not None:
        bl = [bias] if isinstance(bias, torch.Tensor) else list(bias)
    flags = ((_lib.LINEAR_RMS_NORM if gamma is not None else 0) | (_lib.LINEAR_ACCUMULATE if accumulate else 0) |
             (_lib.LINEAR_BIAS if bl is not None else 0) | (_lib.LINEAR_OUT_F16 if out_f16 else 0))
    d = _lib.MxLinearDesc(M=x.shape[0], N=N, K=K, flags=flags, x_stride=x.stride(0), y_stride=outs[0].stride(0),
                          eps=eps, reserved=0)
    need = _lib.linear_workspace_bytes(d)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=x.device) if need else None
    _lib.check(_lib.linear_raw(d, [w.data_ptr() for w in ws_list], x.data_ptr(), [o.data_ptr() for o in outs],
                               gamma.data_ptr() if gamma is not None else 0,
                               None if bl is None else [b.data_ptr() if b is not None else 0 for b in bl],
                               ws.data_ptr() if ws is not None else 0, ws.numel() if ws is not None else 0,
                               _stream()))
    return outs[0] if single else outs


_SA_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}


def self_attention(qkv, *, heads, scale=None, out=None, tuning=None):
    """mx_self_attention, the IR's SelfAttention op: qkv [B][N][3E] contiguous (f32, f16 or bf16) -> y [B][N][E] of the
    same dtype. scale defaults to head_dim^-0.5. The workspace (if the shape needs one) comes from torch's allocator."""
    if not qkv.is_cuda:
        raise ValueError("qkv must be a device tensor")
    if qkv.dim() != 3 or not qkv.is_contiguous() or qkv.dtype not in _SA_DTYPES:
        raise ValueError("qkv must be a contiguous [B][N][3E] f32/f16/bf16 tensor")
    B, N, E3 = qkv.shape
    if E3 % 3:
        raise ValueError("the last dimension of qkv must be a multiple of 3")
    E = E3 // 3
    if scale is None:
        scale = (E // heads) ** -0.5 if heads >= 1 and E % heads == 0 else 1.0
    d = _lib.MxSelfAttnDesc(batch=B, n_tok=N, heads=heads, embed=E, dtype=_SA_DTYPES[qkv.dtype], scale=scale)
    t = _lib.make_tuning(_tuning(tuning))
    if t is not None:
        d.tuning = _lib.ctypes.pointer(t)
    if out is None:
        out = torch.empty(B, N, E, dtype=qkv.dtype, device=qkv.device)
    nbytes = _lib.self_attention_workspace_bytes(d)  # 0 also for an invalid descriptor, which the call reports
    ws = torch.empty(nbytes, dtype=torch.uint8, device=qkv.device) if nbytes else None
    _lib.check(_lib.self_attention_raw(d, qkv.data_ptr(), out.data_ptr(), ws.data_ptr() if ws is not None else 0,
                                       nbytes, _stream()))
    return out
