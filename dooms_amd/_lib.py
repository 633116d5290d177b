"""ctypes binding of libmx_attn.so (the C ABI in include/mx_attn.h).

This is the binding a Python caller of the C ABI would add; it mirrors the reference's own ctypes layer for its C API
(python/dooms/_lib.py:113-229 in dooms.cpp 0.6.1): load the library, declare argument types, turn a non-zero code into
an exception that carries the library's last-error message. There is no fallback: if the library is missing the import
of an entry point raises.
"""
import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libmx_attn.so")

OK = 0
INVALID_ARGUMENT = 1
UNSUPPORTED = 4
RESOURCE_EXHAUSTED = 5
INTERNAL = 7
CODE_NAMES = {OK: "OK", INVALID_ARGUMENT: "INVALID_ARGUMENT", UNSUPPORTED: "UNSUPPORTED",
              RESOURCE_EXHAUSTED: "RESOURCE_EXHAUSTED", INTERNAL: "INTERNAL"}

# Every symbol include/mx_attn.h declares.
EXPORTS = ("mx_attn_abi_version", "mx_attn_last_error", "mx_attn_prefill", "mx_attn_prefill_ws",
           "mx_attn_prefill_workspace_bytes", "mx_attn_prefill_rope", "mx_attn_prefill_rope_ws", "mx_attn_decode",
           "mx_attn_decode_f32", "mx_attn_decode_noalloc", "mx_attn_decode_rope", "mx_linear", "mx_linear_workspace_bytes",
           "mx_attn_decode_workspace_bytes", "mx_attn_decode_workspace_init", "mx_self_attention",
           "mx_self_attention_workspace_bytes")

ROPE_NORMAL = 0  # adjacent pairs (2i, 2i + 1): llama
ROPE_NEOX = 1    # split halves (i, i + head_dim / 2): qwen2
ROPE_NONE = 2    # no rotation: Whisper


class MxAttnTuning(ctypes.Structure):
    """mx_attn_tuning (include/mx_attn.h): 0 in a field keeps the library's plan."""
    _fields_ = [("decode_splits", ctypes.c_int32), ("decode_waves", ctypes.c_int32),
                ("decode_max_workgroups", ctypes.c_int32), ("prefill_plan", ctypes.c_int32),
                ("prefill_stream", ctypes.c_int32)]


class MxAttnDesc(ctypes.Structure):
    """mx_attn_desc (include/mx_attn.h)."""
    _fields_ = [
        ("n_head", ctypes.c_int32), ("n_head_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("n_q", ctypes.c_int32), ("p0", ctypes.c_int32), ("n_kv", ctypes.c_int32), ("causal", ctypes.c_int32),
        ("reserved", ctypes.c_int32), ("q_stride", ctypes.c_int64), ("kv_stride", ctypes.c_int64),
        ("out_stride", ctypes.c_int64), ("scale", ctypes.c_float), ("tuning", ctypes.POINTER(MxAttnTuning)),
    ]


class MxAttnRope(ctypes.Structure):
    """mx_attn_rope (include/mx_attn.h)."""
    _fields_ = [("mode", ctypes.c_int32), ("base", ctypes.c_float)]


class MxLinearDesc(ctypes.Structure):
    """mx_linear_desc (include/mx_linear.h)."""
    _fields_ = [("M", ctypes.c_int32), ("N", ctypes.c_int32), ("K", ctypes.c_int32), ("flags", ctypes.c_uint32),
                ("x_stride", ctypes.c_int64), ("y_stride", ctypes.c_int64), ("eps", ctypes.c_float),
                ("reserved", ctypes.c_int32)]


class MxSelfAttnDesc(ctypes.Structure):
    """mx_self_attn_desc (include/mx_attn.h)."""
    _fields_ = [("batch", ctypes.c_int32), ("n_tok", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("embed", ctypes.c_int32), ("dtype", ctypes.c_int32), ("scale", ctypes.c_float),
                ("tuning", ctypes.POINTER(MxAttnTuning))]


DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2

LINEAR_RMS_NORM, LINEAR_ACCUMULATE, LINEAR_BIAS, LINEAR_OUT_F16 = 1, 2, 4, 8


class MxAttnError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{CODE_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library (raises FileNotFoundError if it was never built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is missing: build it with `python -m dooms_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        L.mx_attn_abi_version.restype = ctypes.c_int32
        L.mx_attn_abi_version.argtypes = []
        L.mx_attn_last_error.restype = ctypes.c_char_p
        L.mx_attn_last_error.argtypes = []
        L.mx_attn_prefill.restype = ctypes.c_int32
        L.mx_attn_prefill.argtypes = [ctypes.POINTER(MxAttnDesc), P, P, P, P, P, P]
        L.mx_attn_prefill_ws.restype = ctypes.c_int32
        L.mx_attn_prefill_ws.argtypes = [ctypes.POINTER(MxAttnDesc), P, P, P, P, P, P, ctypes.c_size_t, P]
        L.mx_attn_prefill_rope_ws.restype = ctypes.c_int32
        L.mx_attn_prefill_rope_ws.argtypes = [ctypes.POINTER(MxAttnDesc), ctypes.POINTER(MxAttnRope), P, P, P, P, P, P,
                                              ctypes.c_size_t, P]
        L.mx_attn_prefill_workspace_bytes.restype = ctypes.c_size_t
        L.mx_attn_prefill_workspace_bytes.argtypes = [ctypes.POINTER(MxAttnDesc)]
        L.mx_attn_decode.restype = ctypes.c_int32
        L.mx_attn_decode.argtypes = [ctypes.POINTER(MxAttnDesc), ctypes.c_int32, ctypes.POINTER(ctypes.c_int32), P,
                                     ctypes.POINTER(P), ctypes.POINTER(P), P, P, P, ctypes.c_size_t, P]
        L.mx_attn_decode_noalloc.restype = ctypes.c_int32
        L.mx_attn_decode_noalloc.argtypes = [ctypes.POINTER(MxAttnDesc), ctypes.c_int32, ctypes.POINTER(ctypes.c_int32),
                                             P, ctypes.POINTER(P), ctypes.POINTER(P), P, P, P]
        L.mx_attn_decode_f32.restype = ctypes.c_int32
        L.mx_attn_decode_f32.argtypes = L.mx_attn_decode.argtypes
        L.mx_attn_prefill_rope.restype = ctypes.c_int32
        L.mx_attn_prefill_rope.argtypes = [ctypes.POINTER(MxAttnDesc), ctypes.POINTER(MxAttnRope), P, P, P, P, P, P]
        L.mx_attn_decode_rope.restype = ctypes.c_int32
        L.mx_attn_decode_rope.argtypes = [ctypes.POINTER(MxAttnDesc), ctypes.POINTER(MxAttnRope), ctypes.c_int32,
                                          ctypes.POINTER(ctypes.c_int32), P, ctypes.POINTER(P), ctypes.POINTER(P), P,
                                          P, P, ctypes.c_size_t, P]
        L.mx_linear_workspace_bytes.restype = ctypes.c_size_t
        L.mx_linear_workspace_bytes.argtypes = [ctypes.POINTER(MxLinearDesc)]
        L.mx_linear.restype = ctypes.c_int32
        L.mx_linear.argtypes = [ctypes.POINTER(MxLinearDesc), ctypes.c_int32, ctypes.POINTER(P), P, ctypes.POINTER(P),
                                P, ctypes.POINTER(P), P, ctypes.c_size_t, P]
        L.mx_attn_decode_workspace_bytes.restype = ctypes.c_size_t
        L.mx_attn_decode_workspace_bytes.argtypes = [ctypes.POINTER(MxAttnDesc), ctypes.c_int32, ctypes.c_int32]
        L.mx_attn_decode_workspace_init.restype = ctypes.c_int32
        L.mx_attn_decode_workspace_init.argtypes = [P, ctypes.c_size_t, P]
        L.mx_self_attention_workspace_bytes.restype = ctypes.c_size_t
        L.mx_self_attention_workspace_bytes.argtypes = [ctypes.POINTER(MxSelfAttnDesc)]
        L.mx_self_attention.restype = ctypes.c_int32
        L.mx_self_attention.argtypes = [ctypes.POINTER(MxSelfAttnDesc), P, P, P, ctypes.c_size_t, P]
        _lib = L
    return _lib


def last_error() -> str:
    return lib().mx_attn_last_error().decode()


def check(code: int) -> None:
    if code != OK:
        raise MxAttnError(code, last_error())


def make_tuning(tuning):
    """An MxAttnTuning from None, an MxAttnTuning or a dict of its fields; None stays None."""
    if tuning is None or isinstance(tuning, MxAttnTuning):
        return tuning
    return MxAttnTuning(**tuning)


def make_desc(n_head, n_head_kv, head_dim, n_q, q_stride, kv_stride, out_stride, scale, p0=0, n_kv=0, causal=1,
              reserved=0, tuning=None) -> MxAttnDesc:
    d = MxAttnDesc(n_head=n_head, n_head_kv=n_head_kv, head_dim=head_dim, n_q=n_q, p0=p0, n_kv=n_kv,
                   causal=causal, reserved=reserved, q_stride=q_stride, kv_stride=kv_stride,
                   out_stride=out_stride, scale=scale)
    t = make_tuning(tuning)
    if t is not None:
        d.tuning = ctypes.pointer(t)
        d._tuning_keepalive = t  # the struct must outlive every call that passes this descriptor
    return d


def prefill_raw(desc: MxAttnDesc, q: int, k: int, v: int, out: int, lse: int, stream: int) -> int:
    """mx_attn_prefill on raw device addresses; returns the code."""
    return lib().mx_attn_prefill(ctypes.byref(desc), q, k, v, out, lse or None, stream or None)


def prefill_ws_raw(desc: MxAttnDesc, q: int, k: int, v: int, out: int, lse: int, ws: int, ws_bytes: int,
                   stream: int) -> int:
    """mx_attn_prefill_ws on raw device addresses; returns the code."""
    return lib().mx_attn_prefill_ws(ctypes.byref(desc), q, k, v, out, lse or None, ws or None, ws_bytes, stream or None)


def prefill_rope_ws_raw(desc: MxAttnDesc, mode: int, base: float, qkv: int, k: int, v: int, out: int, lse: int,
                        ws: int, ws_bytes: int, stream: int) -> int:
    """mx_attn_prefill_rope_ws on raw device addresses; returns the code."""
    rope = MxAttnRope(mode=mode, base=base)
    return lib().mx_attn_prefill_rope_ws(ctypes.byref(desc), ctypes.byref(rope), qkv, k, v, out, lse or None,
                                         ws or None, ws_bytes, stream or None)


def prefill_workspace_bytes(desc: MxAttnDesc) -> int:
    return lib().mx_attn_prefill_workspace_bytes(ctypes.byref(desc))


def decode_raw(desc: MxAttnDesc, kv_len, q: int, k_ptrs, v_ptrs, out: int, lse: int, ws: int, ws_bytes: int,
               stream: int) -> int:
    """mx_attn_decode on raw device addresses; kv_len / k_ptrs / v_ptrs are Python sequences; returns the code."""
    n = len(kv_len)
    lens = (ctypes.c_int32 * n)(*kv_len)
    kp = (ctypes.c_void_p * n)(*k_ptrs)
    vp = (ctypes.c_void_p * n)(*v_ptrs)
    return lib().mx_attn_decode(ctypes.byref(desc), n, lens, q, kp, vp, out, lse or None, ws or None, ws_bytes,
                                stream or None)


def decode_noalloc_raw(desc: MxAttnDesc, kv_len, q: int, k_ptrs, v_ptrs, out: int, lse: int, stream: int) -> int:
    """mx_attn_decode_noalloc on raw device addresses (no workspace: the library's scratch); returns the code."""
    n = len(kv_len)
    lens = (ctypes.c_int32 * n)(*kv_len)
    kp = (ctypes.c_void_p * n)(*k_ptrs)
    vp = (ctypes.c_void_p * n)(*v_ptrs)
    return lib().mx_attn_decode_noalloc(ctypes.byref(desc), n, lens, q, kp, vp, out, lse or None, stream or None)


SCRATCH_BYTES = 16 << 20  # MX_ATTN_SCRATCH_BYTES


def decode_f32_raw(desc: MxAttnDesc, kv_len, q: int, k_ptrs, v_ptrs, out: int, lse: int, ws: int, ws_bytes: int,
                   stream: int) -> int:
    """mx_attn_decode_f32 on raw device addresses; returns the code."""
    n = len(kv_len)
    lens = (ctypes.c_int32 * n)(*kv_len)
    kp = (ctypes.c_void_p * n)(*k_ptrs)
    vp = (ctypes.c_void_p * n)(*v_ptrs)
    return lib().mx_attn_decode_f32(ctypes.byref(desc), n, lens, q, kp, vp, out, lse or None, ws or None, ws_bytes,
                                    stream or None)


def prefill_rope_raw(desc: MxAttnDesc, mode: int, base: float, qkv: int, k: int, v: int, out: int, lse: int,
                     stream: int) -> int:
    """mx_attn_prefill_rope on raw device addresses; returns the code."""
    rope = MxAttnRope(mode=mode, base=base)
    return lib().mx_attn_prefill_rope(ctypes.byref(desc), ctypes.byref(rope), qkv, k, v, out, lse or None,
                                      stream or None)


def decode_rope_raw(desc: MxAttnDesc, mode: int, base: float, kv_len, qkv: int, k_ptrs, v_ptrs, out: int, lse: int,
                    ws: int, ws_bytes: int, stream: int) -> int:
    """mx_attn_decode_rope on raw device addresses; returns the code."""
    n = len(kv_len)
    lens = (ctypes.c_int32 * n)(*kv_len)
    kp = (ctypes.c_void_p * n)(*k_ptrs)
    vp = (ctypes.c_void_p * n)(*v_ptrs)
    rope = MxAttnRope(mode=mode, base=base)
    return lib().mx_attn_decode_rope(ctypes.byref(desc), ctypes.byref(rope), n, lens, qkv, kp, vp, out, lse or None,
                                     ws or None, ws_bytes, stream or None)


def decode_workspace_init(ws: int, ws_bytes: int, stream: int) -> int:
    return lib().mx_attn_decode_workspace_init(ws or None, ws_bytes, stream or None)


def decode_workspace_bytes(desc: MxAttnDesc, batch: int, max_kv_len: int) -> int:
    return lib().mx_attn_decode_workspace_bytes(ctypes.byref(desc), batch, max_kv_len)


def linear_raw(desc: MxLinearDesc, w_ptrs, x: int, y_ptrs, gamma: int, bias_ptrs, ws: int, ws_bytes: int,
               stream: int) -> int:
    """mx_linear on raw device addresses (w_ptrs / y_ptrs / bias_ptrs: Python sequences, bias_ptrs may be None)."""
    n = len(w_ptrs)
    wp = (ctypes.c_void_p * n)(*w_ptrs)
    yp = (ctypes.c_void_p * n)(*y_ptrs)
    bp = None if bias_ptrs is None else (ctypes.c_void_p * n)(*[b or None for b in bias_ptrs])
    return lib().mx_linear(ctypes.byref(desc), n, wp, x, yp, gamma or None, bp, ws or None, ws_bytes, stream or None)


def linear_workspace_bytes(desc: MxLinearDesc) -> int:
    return lib().mx_linear_workspace_bytes(ctypes.byref(desc))


def self_attention_workspace_bytes(desc: MxSelfAttnDesc) -> int:
    return lib().mx_self_attention_workspace_bytes(ctypes.byref(desc))


def self_attention_raw(desc: MxSelfAttnDesc, qkv: int, y: int, ws: int, ws_bytes: int, stream: int) -> int:
    """mx_self_attention on raw device addresses; returns the code."""
    return lib().mx_self_attention(ctypes.byref(desc), qkv, y, ws or None, ws_bytes, stream or None)

