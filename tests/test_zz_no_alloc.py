"""mx_attn_decode_noalloc (the decode entry point that allocates nothing: its workspace is a device array the library
holds) against mx_attn_decode with a caller's workspace, through the C ABI. Both run the same kernels with the same
plan, so the outputs must be bit-identical; two calls in a row, the second with smaller inputs (the array keeps the
first call's state), on both head dims, plus a shape that needs more scratch than the library holds."""
import ctypes
import math

import numpy as np
import pytest
import torch

from dooms_amd import _lib
from dooms_amd import attention as A
from helpers import normal_f16

pytestmark = pytest.mark.gpu


def caches(rng, lens, kvw, device):
    k = [torch.from_numpy(normal_f16(rng, (L, kvw))).to(device) for L in lens]
    v = [torch.from_numpy(normal_f16(rng, (L, kvw))).to(device) for L in lens]
    return k, v


def both(device, rng, n_head, n_kv, hd, lens):
    """(noalloc out, lse), (mx_attn_decode out, lse) for one random problem."""
    B = len(lens)
    q = torch.from_numpy(normal_f16(rng, (B, n_head * hd))).to(device)
    k, v = caches(rng, lens, n_kv * hd, device)
    d = _lib.make_desc(n_head, n_kv, hd, 1, n_head * hd, n_kv * hd, n_head * hd, 1.0 / math.sqrt(hd), causal=0)
    out = torch.full((B, n_head * hd), float("nan"), dtype=torch.float16, device=device)
    lse = torch.full((B, n_head), float("nan"), dtype=torch.float32, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(_lib.decode_noalloc_raw(d, lens, q.data_ptr(), [t.data_ptr() for t in k], [t.data_ptr() for t in v],
                                       out.data_ptr(), lse.data_ptr(), stream))
    ref, rlse = A.decode(q, k, v, lens, n_head=n_head, n_head_kv=n_kv, head_dim=hd, want_lse=True)
    torch.cuda.synchronize()
    return (out.cpu().numpy(), lse.cpu().numpy()), (ref.cpu().numpy(), rlse.cpu().numpy())


def assert_same(a, b, what):
    assert np.array_equal(a[0].view(np.uint16), b[0].view(np.uint16)), f"{what}: outputs differ"
    assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32)), f"{what}: lse differs"


@pytest.mark.parametrize("first,second", [
    ((32, 8, 128, [8192]), (32, 8, 128, [700])),                     # Llama-3-8B: 32 splits, then 6
    ((32, 8, 128, [6841, 1638, 4000, 2721]), (32, 8, 128, [129, 3000])),  # batches
    ((14, 2, 64, [2000]), (14, 2, 64, [513])),                        # Qwen2.5-0.5B
    ((20, 20, 64, [1500] * 5), (20, 20, 64, [448])),                  # Whisper cross (beam 5), then self
])
def test_noalloc_matches_workspace_call(device, first, second):
    rng = np.random.default_rng(sum(first[3]) + len(second[3]))
    for nh, nkv, hd, lens in (first, second):
        got, ref = both(device, rng, nh, nkv, hd, lens)
        assert_same(got, ref, f"{nh}/{nkv} hd {hd} lens {lens}")


def test_noalloc_rejects_beyond_scratch(device):
    # 32 Llama-3-8B sequences at 8192 keys need 17 MB of partials: more than the 16 MiB the library holds
    d = _lib.make_desc(32, 8, 128, 1, 4096, 1024, 4096, 1.0 / math.sqrt(128), causal=0)
    need = _lib.decode_workspace_bytes(d, 32, 8192)
    assert need > _lib.SCRATCH_BYTES
    # buffers that hold the declared shape (one 8192 x 1024 cache shared by every sequence), so that a regression of
    # the size check would compute on valid memory and fail the assertion rather than read out of bounds
    cache = torch.zeros(8192, 1024, dtype=torch.float16, device=device)
    q = torch.zeros(32, 4096, dtype=torch.float16, device=device)
    out = torch.empty_like(q)
    code = _lib.decode_noalloc_raw(d, [8192] * 32, q.data_ptr(), [cache.data_ptr()] * 32, [cache.data_ptr()] * 32,
                                   out.data_ptr(), 0, torch.cuda.current_stream().cuda_stream)
    assert code == _lib.RESOURCE_EXHAUSTED and "scratch" in _lib.last_error()


def test_noalloc_two_streams_ordered_by_caller(device):
    """Calls on two streams share the GPU's one array; the contract is that the caller orders them. Two calls in a row
    on two streams, the second made to wait for the first with an event, each match mx_attn_decode bit for bit."""
    rng = np.random.default_rng(11)
    n_head, n_kv, hd = 32, 8, 128
    d = _lib.make_desc(n_head, n_kv, hd, 1, n_head * hd, n_kv * hd, n_head * hd, 1.0 / math.sqrt(hd), causal=0)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    probs = []
    for lens in ([8192], [3000, 129]):
        B = len(lens)
        q = torch.from_numpy(normal_f16(rng, (B, n_head * hd))).to(device)
        k, v = caches(rng, lens, n_kv * hd, device)
        out = torch.full((B, n_head * hd), float("nan"), dtype=torch.float16, device=device)
        probs.append((lens, q, k, v, out))
    torch.cuda.synchronize()
    ev = torch.cuda.Event()
    for (lens, q, k, v, out), st in zip(probs, (s1, s2)):
        if st is s2:
            st.wait_event(ev)
        _lib.check(_lib.decode_noalloc_raw(d, lens, q.data_ptr(), [t.data_ptr() for t in k], [t.data_ptr() for t in v],
                                           out.data_ptr(), 0, st.cuda_stream))
        if st is s1:
            ev.record(s1)
    torch.cuda.synchronize()
    for lens, q, k, v, out in probs:
        ref, _ = A.decode(q, k, v, lens, n_head=n_head, n_head_kv=n_kv, head_dim=hd)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.cpu().numpy().view(np.uint16)), lens
