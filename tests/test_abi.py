"""The C ABI (include/mx_attn.h, dooms_amd/libmx_attn.so) on the CPU: the library loads, exports exactly what the header
declares, the descriptor layout agrees between C and the binding, and every argument check returns the documented code
(the dooms_code numbering, include/dooms/dooms_c.h:24-33 in the reference) with a message, before anything touches a GPU.
"""
import ctypes
import glob
import os
import re
import subprocess
import threading

import pytest

from dooms_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mx_attn.h")
A = 256  # a 256-byte aligned fake device address: never dereferenced, every call below fails its checks first


HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared():
    text = "".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"MX_ATTN_API\s+[\w\s\*]+?\b(mx_\w+)\s*\(", text)))


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    return sorted(l.split()[-1] for l in out.splitlines() if " T " in l)


def test_library_loads():
    assert _lib.lib().mx_attn_abi_version() == 3


def test_exports_exactly_the_header():
    assert declared() == sorted(_lib.EXPORTS)
    assert exported() == declared()


def test_desc_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "mx_attn.h"\n'
                   'int main(void){printf("%zu %zu %zu %zu %zu\\n", sizeof(mx_attn_desc), offsetof(mx_attn_desc, reserved),'
                   ' offsetof(mx_attn_desc, q_stride), offsetof(mx_attn_desc, out_stride), offsetof(mx_attn_desc, scale));'
                   'printf("%zu %zu %zu %zu %zu\\n", offsetof(mx_attn_desc, tuning), sizeof(mx_attn_tuning),'
                   ' offsetof(mx_attn_tuning, prefill_plan), offsetof(mx_attn_tuning, prefill_stream),'
                   ' offsetof(mx_self_attn_desc, tuning));'
                   'return 0;}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)],
                   check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    D = _lib.MxAttnDesc
    T, S = _lib.MxAttnTuning, _lib.MxSelfAttnDesc
    assert got == [ctypes.sizeof(D), D.reserved.offset, D.q_stride.offset, D.out_stride.offset, D.scale.offset,
                   D.tuning.offset, ctypes.sizeof(T), T.prefill_plan.offset, T.prefill_stream.offset, S.tuning.offset]


def desc(**kw):
    base = dict(n_head=32, n_head_kv=8, head_dim=128, n_q=1, q_stride=4096, kv_stride=1024, out_stride=4096,
                scale=0.0883883)
    base.update(kw)
    return _lib.make_desc(**base)


def prefill(d, q=A, k=A, v=A, out=A, lse=0):
    return _lib.lib().mx_attn_prefill(ctypes.byref(d) if d is not None else None, q, k, v, out, lse or None, None)


def decode(d, lens=(100,), kp=None, vp=None, q=A, out=A, lse=0, ws=A, ws_bytes=1 << 30, batch=None):
    n = len(lens)
    L = (ctypes.c_int32 * max(n, 1))(*lens)
    K = (ctypes.c_void_p * max(n, 1))(*(kp or [A] * n))
    V = (ctypes.c_void_p * max(n, 1))(*(vp or [A] * n))
    return _lib.lib().mx_attn_decode(ctypes.byref(d), n if batch is None else batch, L, q, K, V, out, lse or None,
                                     ws or None, ws_bytes, None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(reserved=1), _lib.INVALID_ARGUMENT, "reserved"),
    (dict(n_head=0), _lib.INVALID_ARGUMENT, "n_head"),
    (dict(n_head=14, n_head_kv=3), _lib.INVALID_ARGUMENT, "multiple"),
    (dict(head_dim=0), _lib.INVALID_ARGUMENT, "head_dim"),
    (dict(head_dim=80, q_stride=2560, kv_stride=640, out_stride=2560), _lib.UNSUPPORTED, "not supported"),
    (dict(head_dim=96, q_stride=3072, kv_stride=768, out_stride=3072), _lib.UNSUPPORTED, "not supported"),
    (dict(head_dim=2, q_stride=64, kv_stride=16, out_stride=64), _lib.UNSUPPORTED, "power of two"),
    (dict(head_dim=512, q_stride=16384, kv_stride=4096, out_stride=16384), _lib.UNSUPPORTED, "power of two"),
    (dict(head_dim=4, n_head_kv=1, n_head=4, q_stride=16, kv_stride=6, out_stride=16), _lib.INVALID_ARGUMENT,
     "multiples of 4"),
    (dict(head_dim=16, n_head=4, n_head_kv=2, q_stride=68, kv_stride=32, out_stride=64), _lib.INVALID_ARGUMENT,
     "multiples of 8"),
    (dict(n_q=-1), _lib.INVALID_ARGUMENT, "n_q"),
    (dict(causal=2), _lib.INVALID_ARGUMENT, "causal"),
    (dict(scale=float("nan")), _lib.INVALID_ARGUMENT, "scale"),
    (dict(scale=float("inf")), _lib.INVALID_ARGUMENT, "scale"),
    (dict(q_stride=4088), _lib.INVALID_ARGUMENT, "q_stride"),
    (dict(kv_stride=1016), _lib.INVALID_ARGUMENT, "kv_stride"),
    (dict(out_stride=100), _lib.INVALID_ARGUMENT, "out_stride"),
    (dict(q_stride=4100), _lib.INVALID_ARGUMENT, "multiples of 8"),
    (dict(tuning=dict(decode_splits=65)), _lib.INVALID_ARGUMENT, "decode_splits"),
    (dict(tuning=dict(decode_splits=-1)), _lib.INVALID_ARGUMENT, "decode_splits"),
    (dict(tuning=dict(decode_waves=6)), _lib.INVALID_ARGUMENT, "decode_waves"),
    (dict(tuning=dict(decode_max_workgroups=-2)), _lib.INVALID_ARGUMENT, "decode_max_workgroups"),
    (dict(tuning=dict(prefill_plan=3)), _lib.INVALID_ARGUMENT, "prefill_plan"),
    (dict(tuning=dict(prefill_stream=2)), _lib.INVALID_ARGUMENT, "prefill_stream"),
    (dict(tuning=dict(prefill_stream=-2)), _lib.INVALID_ARGUMENT, "prefill_stream"),
])
def test_descriptor_checks(kw, code, msg):
    for call in (lambda d: prefill(d), lambda d: decode(d)):
        assert call(desc(**kw)) == code
        assert msg in _lib.last_error()


def test_null_descriptor():
    assert prefill(None) == _lib.INVALID_ARGUMENT
    assert "desc is null" in _lib.last_error()


def test_prefill_checks():
    assert prefill(desc(p0=-1)) == _lib.INVALID_ARGUMENT and "p0" in _lib.last_error()
    assert prefill(desc(n_kv=-1)) == _lib.INVALID_ARGUMENT
    assert prefill(desc(n_q=10, p0=5, n_kv=12)) == _lib.INVALID_ARGUMENT and "n_kv" in _lib.last_error()
    assert prefill(desc(), q=0) == _lib.INVALID_ARGUMENT and "null" in _lib.last_error()
    assert prefill(desc(), out=A + 2) == _lib.INVALID_ARGUMENT and "aligned" in _lib.last_error()
    assert prefill(desc(), lse=A + 2) == _lib.INVALID_ARGUMENT and "lse" in _lib.last_error()
    # zero rows: nothing to do, no pointer is looked at
    assert prefill(desc(n_q=0), q=0, k=0, v=0, out=0) == _lib.OK


def test_decode_checks():
    d = desc()
    assert decode(d, batch=0) == _lib.INVALID_ARGUMENT and "batch" in _lib.last_error()
    assert decode(d, lens=(100, 0)) == _lib.INVALID_ARGUMENT and "kv_len[1]" in _lib.last_error()
    assert decode(desc(n_q=8, causal=1), lens=(5,)) == _lib.INVALID_ARGUMENT and "n_q" in _lib.last_error()
    assert decode(d, lens=(100, 100), kp=[A, 0]) == _lib.INVALID_ARGUMENT and "sequence 1" in _lib.last_error()
    assert decode(d, lens=(100,), vp=[A + 8]) == _lib.INVALID_ARGUMENT and "aligned" in _lib.last_error()
    assert decode(d, q=0) == _lib.INVALID_ARGUMENT
    assert decode(d, lens=(5000,), ws_bytes=16) == _lib.RESOURCE_EXHAUSTED and "workspace" in _lib.last_error()
    assert decode(d, lens=(5000,), ws=0) == _lib.INVALID_ARGUMENT and "workspace is null" in _lib.last_error()
    assert decode(d, lens=(5000,), ws=A + 16) == _lib.INVALID_ARGUMENT and "256-byte" in _lib.last_error()
    assert decode(desc(n_q=0), lens=(5,)) == _lib.OK
    # (kv head, row tile) pairs of one sequence beyond the 2048 one launch holds: refused before anything is enqueued
    assert decode(desc(n_q=40000, causal=0), lens=(100,)) == _lib.UNSUPPORTED and "too large" in _lib.last_error()
    assert decode(desc(n_q=1025, causal=0), lens=(100,)) == _lib.UNSUPPORTED  # 8 kv heads x 257 tiles of 16 rows


def rope_decode(d, mode=0, base=500000.0, lens=(100,), kp=None, vp=None, qkv=A, rope=True):
    n = len(lens)
    L = (ctypes.c_int32 * n)(*lens)
    K = (ctypes.c_void_p * n)(*(kp or [A + 4096 * i for i in range(n)]))
    V = (ctypes.c_void_p * n)(*(vp or [A + 65536 + 4096 * i for i in range(n)]))
    r = _lib.MxAttnRope(mode=mode, base=base)
    return _lib.lib().mx_attn_decode_rope(ctypes.byref(d), ctypes.byref(r) if rope else None, n, L, qkv, K, V, A, None,
                                          A, 1 << 30, None)


def test_decode_rope_checks():
    d = desc(q_stride=6144)  # (32 + 2 * 8) * 128
    assert rope_decode(d, rope=False) == _lib.INVALID_ARGUMENT and "rope is null" in _lib.last_error()
    assert rope_decode(d, mode=3) == _lib.INVALID_ARGUMENT and "mode" in _lib.last_error()
    assert rope_decode(d, base=0.0) == _lib.INVALID_ARGUMENT and "base" in _lib.last_error()
    assert rope_decode(d, base=float("nan")) == _lib.INVALID_ARGUMENT and "base" in _lib.last_error()
    assert rope_decode(desc(q_stride=4096)) == _lib.INVALID_ARGUMENT and "q_stride" in _lib.last_error()
    assert rope_decode(desc(q_stride=6144, n_q=2)) == _lib.INVALID_ARGUMENT and "n_q" in _lib.last_error()
    assert rope_decode(d, lens=(5, 6), kp=[A, A]) == _lib.INVALID_ARGUMENT and "share a cache" in _lib.last_error()
    assert rope_decode(d, lens=(5, 0)) == _lib.INVALID_ARGUMENT and "kv_len[1]" in _lib.last_error()
    assert rope_decode(d, qkv=A + 8) == _lib.INVALID_ARGUMENT and "aligned" in _lib.last_error()


def test_prefill_rope_checks():
    L = _lib.lib()
    r = _lib.MxAttnRope(mode=1, base=1e6)
    call = lambda d, rope=r, qkv=A: L.mx_attn_prefill_rope(ctypes.byref(d), ctypes.byref(rope) if rope else None, qkv,
                                                           A, A, A, None, None)
    d = desc(q_stride=6144, n_q=16, p0=4)
    assert call(d, rope=None) == _lib.INVALID_ARGUMENT and "rope is null" in _lib.last_error()
    assert call(d, rope=_lib.MxAttnRope(mode=-1, base=1.0)) == _lib.INVALID_ARGUMENT
    assert call(desc(q_stride=4096, n_q=16)) == _lib.INVALID_ARGUMENT and "q_stride" in _lib.last_error()
    assert call(desc(q_stride=6144, n_q=16, p0=4, n_kv=10, causal=0)) == _lib.INVALID_ARGUMENT
    assert "cache" in _lib.last_error()
    assert call(d, qkv=A + 4) == _lib.INVALID_ARGUMENT and "aligned" in _lib.last_error()
    assert call(desc(q_stride=6144, n_q=0)) == _lib.OK


def test_workspace_init_checks():
    L = _lib.lib()
    assert L.mx_attn_decode_workspace_init(None, 0, None) == _lib.OK
    assert L.mx_attn_decode_workspace_init(None, 256, None) == _lib.INVALID_ARGUMENT
    assert L.mx_attn_decode_workspace_init(A + 4, 256, None) == _lib.INVALID_ARGUMENT


def test_workspace_size():
    d = desc()
    ws = lambda b, n: _lib.decode_workspace_bytes(d, b, n)
    assert ws(1, 1) == 0 and ws(1, 128) == 0  # one split: no partials
    assert ws(1, 129) > 0
    assert ws(1, 8192) <= ws(1, 8193) <= ws(4, 8193) <= ws(32, 8193) == ws(100, 8193)  # launches of 32 reuse it
    # the fixed counter region (2048 lines of 256 bytes), plus min(8192/128, 32) = 32 splits x 8 kv heads x 4 rows x
    # (128 + 4) floats
    assert ws(1, 8192) == 2048 * 256 + 32 * 8 * 4 * 132 * 4
    assert ws(1, 4096) == ws(1, 8192) and ws(1, 2048) == 2048 * 256 + 16 * 8 * 4 * 132 * 4
    assert _lib.decode_workspace_bytes(desc(n_head=3, n_head_kv=2), 1, 1000) == 0
    assert "multiple" in _lib.last_error()


def test_prefill_ws_checks():
    # the split-KV route for chunks of few rows: a decode workspace sized for the chunk's rows over p0 + n_q keys
    d16 = desc(n_head=28, n_head_kv=4, n_q=16, p0=30000, q_stride=3584, kv_stride=512, out_stride=3584)
    n = _lib.prefill_workspace_bytes(d16)  # 16 x 7 rows: 7 row tiles of 16 per kv head
    # the decode workspace (the counter region, 32 splits of partials), then room for the rotated f32 query rows of the
    # rope call
    assert n == 2048 * 256 + 32 * 4 * 7 * 16 * 132 * 4 + 16 * 28 * 128 * 4
    # a 2048-row chunk of 28 heads: 224 tiles of the 8-wave grid for 256 CUs. At head dim 64, behind a prefix at least
    # as long as the chunk, the stream-K split of the 8-wave plan is planned; its workspace is the counter region, then
    # 2 partial slots per range (256 ranges) of 8 waves x 64 lanes x (32 + 2) floats. The same chunk as a whole prompt
    # (p0 0) runs the 4-wave grid (no workspace). At head dim 128 the grid runs (no workspace) unless the tuning forces
    # the split.
    big64 = desc(n_head=28, n_head_kv=4, head_dim=64, n_q=2048, p0=2048, q_stride=1792, kv_stride=256, out_stride=1792)
    assert _lib.prefill_workspace_bytes(big64) == 2048 * 256 + 512 * 8 * 64 * 34 * 4
    first64 = desc(n_head=28, n_head_kv=4, head_dim=64, n_q=2048, p0=0, q_stride=1792, kv_stride=256, out_stride=1792)
    assert _lib.prefill_workspace_bytes(first64) == 0
    big = desc(n_head=28, n_head_kv=4, n_q=2048, p0=0, q_stride=3584, kv_stride=512, out_stride=3584)
    assert _lib.prefill_workspace_bytes(big) == 0
    forced = desc(n_head=28, n_head_kv=4, n_q=2048, p0=0, q_stride=3584, kv_stride=512, out_stride=3584,
                  tuning=dict(prefill_stream=1))
    assert _lib.prefill_workspace_bytes(forced) == 2048 * 256 + 512 * 8 * 64 * 66 * 4
    off = desc(n_head=28, n_head_kv=4, head_dim=64, n_q=2048, p0=0, q_stride=1792, kv_stride=256, out_stride=1792,
               tuning=dict(prefill_stream=-1))
    assert _lib.prefill_workspace_bytes(off) == 0  # the flash kernel's own grid, no workspace
    # a causal 4096-token prompt at head dim 64 (no prefix: the 4-wave grid), of 14 heads or of 32: no workspace
    assert _lib.prefill_workspace_bytes(desc(n_head=14, n_head_kv=2, head_dim=64, n_q=4096, q_stride=896,
                                             kv_stride=128, out_stride=896)) == 0
    assert _lib.prefill_workspace_bytes(desc(n_head=32, n_head_kv=8, head_dim=64, n_q=4096, q_stride=2048,
                                             kv_stride=512, out_stride=2048)) == 0
    # 256 equal tiles (non-causal, 2048 rows of 32 heads): one full round of the grid, nothing to balance
    even = desc(n_head=32, n_head_kv=8, n_q=2048, p0=0, n_kv=4096, causal=0, q_stride=4096, kv_stride=1024,
                out_stride=4096)
    assert _lib.prefill_workspace_bytes(even) == 0
    assert _lib.prefill_workspace_bytes(desc(n_head=32, n_head_kv=8, n_q=2048, p0=0, n_kv=4096, causal=0,
                                             q_stride=4096, kv_stride=1024, out_stride=4096,
                                             tuning=dict(prefill_stream=1))) == 2048 * 256 + 512 * 8 * 64 * 66 * 4
    assert _lib.prefill_workspace_bytes(desc(n_head=3, n_head_kv=2)) == 0 and "multiple" in _lib.last_error()
    call = lambda d, ws=A, nb=1 << 40: _lib.prefill_ws_raw(d, A, A, A, A, 0, ws, nb, 0)
    n_dec = n - 16 * 28 * 128 * 4  # mx_attn_prefill_ws itself needs only the decode part
    assert call(d16, nb=n_dec - 1) == _lib.RESOURCE_EXHAUSTED and "workspace" in _lib.last_error()
    assert call(d16, ws=A + 16) == _lib.INVALID_ARGUMENT and "256-byte" in _lib.last_error()
    bad = desc(n_head=28, n_head_kv=4, n_q=16, p0=100, n_kv=50, q_stride=3584, kv_stride=512, out_stride=3584)
    assert call(bad) == _lib.INVALID_ARGUMENT and "n_kv" in _lib.last_error()
    assert call(desc(n_head=28, n_head_kv=4, n_q=16, p0=-1, q_stride=3584, kv_stride=512, out_stride=3584)) == \
        _lib.INVALID_ARGUMENT
    # the rope variant: the same workspace, its tail holding the rotated f32 query rows
    dr = desc(n_head=28, n_head_kv=4, n_q=16, p0=30000, q_stride=4608, kv_stride=512, out_stride=3584)
    nr = _lib.prefill_workspace_bytes(dr)
    assert nr == n
    rcall = lambda d, ws=A, nb=1 << 40: _lib.prefill_rope_ws_raw(d, 0, 500000.0, A, A, A, A, 0, ws, nb, 0)
    assert rcall(dr, nb=nr - 1) == _lib.RESOURCE_EXHAUSTED and "workspace" in _lib.last_error()
    assert rcall(dr, ws=A + 16) == _lib.INVALID_ARGUMENT and "256-byte" in _lib.last_error()
    assert rcall(desc(n_head=28, n_head_kv=4, n_q=16, q_stride=3584, kv_stride=512, out_stride=3584)) == \
        _lib.INVALID_ARGUMENT and "q_stride" in _lib.last_error()


def test_last_error_is_per_thread():
    prefill(desc(head_dim=80))
    assert "not supported" in _lib.last_error()
    seen = []
    t = threading.Thread(target=lambda: seen.append(_lib.last_error()))
    t.start()
    t.join()
    assert seen == [""]


def test_python_front_end_refuses_host_tensors():
    import torch
    from dooms_amd import attention
    x = torch.zeros(4, 128, dtype=torch.float16)
    with pytest.raises(ValueError):
        attention.prefill(x, x, x, n_head=1, n_head_kv=1, head_dim=128)


def test_linear_desc_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "mx_linear.h"\n'
                   'int main(void){printf("%zu %zu %zu %zu %zu\\n", sizeof(mx_linear_desc), offsetof(mx_linear_desc, flags),'
                   ' offsetof(mx_linear_desc, x_stride), offsetof(mx_linear_desc, eps), offsetof(mx_linear_desc, reserved));'
                   'return 0;}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)],
                   check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    D = _lib.MxLinearDesc
    assert got == [ctypes.sizeof(D), D.flags.offset, D.x_stride.offset, D.eps.offset, D.reserved.offset]


def test_linear_checks():
    def ld(**kw):
        base = dict(M=4, N=64, K=128, flags=0, x_stride=128, y_stride=64, eps=1e-5, reserved=0)
        base.update(kw)
        return _lib.MxLinearDesc(**base)

    def call(d, count=1, w=A, x=A, y=A, gamma=0, bias=None, ws=0, ws_bytes=0):
        return _lib.linear_raw(d, [w] * count, x, [y] * count, gamma, bias, ws, ws_bytes, 0)

    assert call(ld(K=100, x_stride=100)) == _lib.UNSUPPORTED and "multiple of 32" in _lib.last_error()
    assert call(ld(reserved=1)) == _lib.INVALID_ARGUMENT
    assert call(ld(flags=16)) == _lib.INVALID_ARGUMENT and "flags" in _lib.last_error()
    assert call(ld(x_stride=64)) == _lib.INVALID_ARGUMENT and "x_stride" in _lib.last_error()
    assert call(ld(y_stride=66)) == _lib.INVALID_ARGUMENT and "y_stride" in _lib.last_error()
    assert call(ld(flags=8, y_stride=68)) == _lib.INVALID_ARGUMENT  # f16 rows need a multiple of 8
    assert call(ld(), count=0) == _lib.INVALID_ARGUMENT and "count" in _lib.last_error()
    assert call(ld(), count=65) == _lib.INVALID_ARGUMENT
    assert call(ld(flags=1)) == _lib.INVALID_ARGUMENT and "gamma" in _lib.last_error()
    assert call(ld(flags=4)) == _lib.INVALID_ARGUMENT and "bias" in _lib.last_error()
    assert call(ld(), x=A + 4) == _lib.INVALID_ARGUMENT and "aligned" in _lib.last_error()
    # the GEMM path (M > 8) stages the input rows as half: M * K halves of workspace
    d = ld(M=100, flags=1)
    assert _lib.linear_workspace_bytes(d) == 100 * 128 * 2 and _lib.linear_workspace_bytes(ld(M=8, flags=1)) == 0
    assert _lib.linear_workspace_bytes(ld(M=9, K=96, x_stride=96)) == 2304  # 9 rows x 128 padded columns x 2 bytes
    assert call(d, gamma=A, ws=A, ws_bytes=256) == _lib.RESOURCE_EXHAUSTED
    assert call(d, gamma=A, ws=A + 16, ws_bytes=1 << 20) == _lib.INVALID_ARGUMENT
    assert call(ld(M=100)) == _lib.INVALID_ARGUMENT and "workspace" in _lib.last_error()
    assert call(ld(M=0), w=0, x=0, y=0) == _lib.OK


def test_self_attn_desc_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "mx_attn.h"\n'
                   'int main(void){printf("%zu %zu %zu\\n", sizeof(mx_self_attn_desc), offsetof(mx_self_attn_desc, dtype),'
                   ' offsetof(mx_self_attn_desc, scale));return 0;}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)],
                   check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    D = _lib.MxSelfAttnDesc
    assert got == [ctypes.sizeof(D), D.dtype.offset, D.scale.offset]


def test_self_attention_checks():
    """Argument checks of mx_self_attention, with the reference's own messages where it has them
    (self_attention_params, src/ir/op.cpp:69-76; infer_self_attention, src/ir/shape_infer.cpp:156-171)."""
    def sd(**kw):
        base = dict(batch=1, n_tok=210, heads=16, embed=1280, dtype=_lib.DTYPE_F32, scale=80 ** -0.5)
        base.update(kw)
        return _lib.MxSelfAttnDesc(**base)

    def call(d, qkv=A, y=1 << 40, ws=A, ws_bytes=1 << 30):
        return _lib.self_attention_raw(d, qkv, y, ws, ws_bytes, 0)

    assert call(sd(heads=0)) == _lib.INVALID_ARGUMENT and "heads must be >= 1" in _lib.last_error()
    assert call(sd(heads=3)) == _lib.INVALID_ARGUMENT and "not divisible by 3 heads" in _lib.last_error()
    assert call(sd(scale=float("inf"))) == _lib.INVALID_ARGUMENT and "scale must be finite" in _lib.last_error()
    assert call(sd(dtype=3)) == _lib.INVALID_ARGUMENT and "dtype" in _lib.last_error()
    assert call(sd(batch=0)) == _lib.INVALID_ARGUMENT
    assert call(sd(heads=4, embed=4 * 160)) == _lib.UNSUPPORTED and "head_dim 160" in _lib.last_error()
    assert call(sd(), qkv=0) == _lib.INVALID_ARGUMENT and "null" in _lib.last_error()
    assert call(sd(), qkv=A + 4) == _lib.INVALID_ARGUMENT and "aligned" in _lib.last_error()
    assert call(sd(), y=A) == _lib.INVALID_ARGUMENT and "overlaps" in _lib.last_error()
    assert call(sd(n_tok=0), qkv=0, y=0) == _lib.OK
    # workspace: none when head_dim is a multiple of 8 (the rows are read in place, any dtype), padded operands otherwise
    for dt in (_lib.DTYPE_F32, _lib.DTYPE_F16, _lib.DTYPE_BF16):
        assert _lib.self_attention_workspace_bytes(sd(heads=20, dtype=dt)) == 0  # head_dim 64
        assert _lib.self_attention_workspace_bytes(sd(dtype=dt)) == 0            # ViT-H: head_dim 80
    w = 210 * 16 * 64  # head_dim 6 padded to 64: f32 Q, f16 K and V, f32 O
    odd = sd(embed=16 * 6)
    assert _lib.self_attention_workspace_bytes(odd) == w * 4 + w * 2 * 2 + w * 4
    n = _lib.self_attention_workspace_bytes(odd)
    assert call(odd, ws_bytes=n - 1) == _lib.RESOURCE_EXHAUSTED
    assert call(odd, ws=0, ws_bytes=n) == _lib.INVALID_ARGUMENT
    assert call(odd, ws=A + 16, ws_bytes=n) == _lib.INVALID_ARGUMENT and "256-byte" in _lib.last_error()


def test_host_code_under_address_and_undefined_behaviour_sanitizers():
    """The library's host code (every .hip source's host side, device code unchanged) built with -fsanitize=address,
    undefined and driven through every entry point's argument checks and the workspace-size arithmetic over many
    shapes (tests/cpp/abi_checks_sanitized.cpp). No GPU needed: every call is refused before anything is enqueued."""
    from dooms_amd import build as B
    exe = os.path.join(B.SAN_DIR, "abi_checks_sanitized")
    srcs = [os.path.join(B.CSRC, s) for s in os.listdir(B.CSRC)] + glob.glob(os.path.join(ROOT, "include", "*.h")) + \
        [os.path.join(ROOT, "tests", "cpp", "abi_checks_sanitized.cpp")]
    if not os.path.exists(exe) or os.path.getmtime(exe) < max(os.path.getmtime(s) for s in srcs):
        exe = B.build_sanitized_abi_check()
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300,
                       env={**os.environ, "ASAN_OPTIONS": "detect_leaks=0"})  # the HIP runtime's own allocations
    assert r.returncode == 0, r.stdout + r.stderr
    assert "abi_checks_sanitized: ok" in r.stdout


def test_stream_k_partition(tmp_path):
    # the stream-K prefill's partition arithmetic (mx_kernels.hpp), checked on the CPU over many launch shapes by
    # tests/cpp/sk_partition_check.cpp: every unit in exactly one segment, each split tile's slots where its merge reads
    exe = tmp_path / "sk_partition_check"
    src = os.path.join(ROOT, "tests", "cpp", "sk_partition_check.cpp")
    subprocess.run(["/opt/rocm/bin/hipcc", "-O2", "-std=c++17", "--offload-arch=gfx950",
                    "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "dooms_amd", "csrc"), src,
                    "-o", str(exe)], check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout
    assert "0 failures" in r.stdout
