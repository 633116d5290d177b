"""dooms_amd: the attention hot path of dooms.cpp (causal GQA prefill flash attention and KV-cache decode attention)
as hand-written HIP kernels for MI355X (gfx950) behind a C ABI (include/mx_attn.h, libmx_attn.so)."""
from ._lib import MxAttnError, LIB_PATH, EXPORTS  # noqa: F401

__all__ = ["MxAttnError", "LIB_PATH", "EXPORTS"]
