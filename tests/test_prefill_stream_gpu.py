"""Parity of the stream-K prefill (mx_attn_prefill_ws / mx_attn_prefill_rope_ws on the 8-wave plan) with the f64 oracle
and with the one-tile-per-workgroup grid of mx_attn_prefill, through the C ABI.

Reference: attention_prefill<64|128> (llama_kernels.h:632-769) for a prompt chunk (metal_llama_decoder.mm:284-296). The
stream-K split is this library's own scheduling: every CU takes an equal range of (query tile, 64-key block) units and
a tile split between ranges is merged with the log-sum-exp rule, so results agree with the grid within the tolerance
(the summation order differs) and are reproducible bit for bit from call to call.
"""
import numpy as np
import pytest
import torch

from dooms_amd import _lib
from dooms_amd import attention as A
from helpers import assert_close, normal_f16, ref_attention

pytestmark = pytest.mark.gpu


def inputs(device, seed, n_q, n_kv, n_head, n_head_kv, hd, sigma=0.5):
    rng = np.random.default_rng(seed)
    q = normal_f16(rng, (n_q, n_head * hd), sigma)
    k = normal_f16(rng, (n_kv, n_head_kv * hd), sigma)
    v = normal_f16(rng, (n_kv, n_head_kv * hd), sigma)
    return q, k, v, [torch.from_numpy(a).to(device) for a in (q, k, v)]


def ws_bytes(n_q, n_head, n_head_kv, hd, p0, n_kv, causal, tuning):
    d = _lib.make_desc(n_head, n_head_kv, hd, n_q, n_head * hd, n_head_kv * hd, n_head * hd, 1.0 / np.sqrt(hd),
                       p0=p0, n_kv=n_kv, causal=int(causal), tuning=tuning)
    return _lib.prefill_workspace_bytes(d)


def run_case(device, seed, n_q, p0, n_head, n_head_kv, hd, causal=True, extra=0, forced=False, rows=None, heads=None):
    """The chunk's rows at p0 over p0 + n_q + extra keys: stream-K (workspace) against the grid and the oracle. forced:
    the 8-wave plan and its stream-K split fixed by the tuning (shapes that the planner would give other plans)."""
    n_kv = p0 + n_q + extra
    tuning = dict(prefill_plan=8, prefill_stream=1) if forced else None
    nb = ws_bytes(n_q, n_head, n_head_kv, hd, p0, n_kv, causal, tuning)
    assert nb > 0, "the case must take the stream-K plan"
    q, k, v, (dq, dk, dv) = inputs(device, seed, n_q, n_kv, n_head, n_head_kv, hd)
    kw = dict(n_head=n_head, n_head_kv=n_head_kv, head_dim=hd, p0=p0, n_kv=n_kv, causal=causal, want_lse=True)
    grid, lgrid = A.prefill(dq, dk, dv, tuning=dict(prefill_plan=8) if forced else None, **kw)
    ws = A.new_workspace(nb, device)
    sk, lsk = A.prefill(dq, dk, dv, workspace=ws, tuning=tuning, **kw)
    sk2, lsk2 = A.prefill(dq, dk, dv, workspace=ws, tuning=tuning, **kw)  # the counters are back at 0
    torch.cuda.synchronize()
    assert torch.equal(sk, sk2) and torch.equal(lsk, lsk2), "stream-K is reproducible call to call"
    assert not torch.isnan(sk).any()
    # against the grid: the same math in another summation order (f16 outputs: a few ulps)
    np.testing.assert_allclose(sk.cpu().float().numpy(), grid.cpu().float().numpy(), atol=2e-3, rtol=0)
    np.testing.assert_allclose(lsk.cpu().numpy(), lgrid.cpu().numpy(), atol=1e-4, rtol=1e-5)
    rows = np.arange(n_q) if rows is None else np.asarray(rows)
    heads = np.arange(n_head) if heads is None else np.asarray(heads)
    ro, rl = ref_attention(q, k, v, n_head, n_head_kv, hd, 1.0 / np.sqrt(hd), p0=p0, causal=causal, rows=rows,
                           heads=heads)
    cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
    assert_close(sk.cpu().numpy().astype(np.float64)[rows][:, cols], ro, hd, f"stream-K n_q={n_q} p0={p0}",
                 lsk.cpu().numpy()[rows][:, heads], rl)


def test_qwen7b_chunk(device):
    # a 2048-row chunk of Qwen2.5-7B at p0 = 6144: 224 tiles for 256 CUs, split over all 256; every head of sampled rows
    rows = [0, 1, 255, 256, 1000, 1023, 1024, 2046, 2047]
    run_case(device, 1, 2048, 6144, 28, 4, 128, forced=True, rows=rows)


def test_qwen05b_chunk_planned(device):
    # a 2048-row Qwen2.5-0.5B chunk behind a 4096-token prefix (head dim 64, 112 tiles of the 8-wave grid): the planner
    # takes the split
    run_case(device, 8, 2048, 4096, 14, 2, 64, rows=list(range(0, 2048, 37)) + [2047])


@pytest.mark.parametrize("n_q,p0,nh,nkv", [(128, 4000, 28, 4), (447, 7648, 8, 2)])
def test_fewer_ranges_than_cus(device, n_q, p0, nh, nkv):
    # launches of fewer than 8 blocks per CU: the split takes fewer ranges (224 and 248, multiples of 8, each dealt to
    # exactly one workgroup); the second shape ran 250 ranges, two of them on one workgroup and one on none, before the
    # plan rounded the count to a multiple of 8
    run_case(device, 9, n_q, p0, nh, nkv, 128, rows=list(range(0, n_q, 11)) + [n_q - 1])


def test_many_ranges_per_tile(device):
    # 2 query tiles x 8 heads of ~136 blocks over 256 ranges of ~8.5 blocks: each tile is merged from ~16 slots
    run_case(device, 2, 512, 8192, 8, 2, 128, forced=True, rows=list(range(0, 512, 7)) + [511])


def test_head_dim_64_ragged(device):
    # head dim 64, a ragged last query tile (700 rows) and cache rows past the chunk (masked by causality)
    run_case(device, 3, 700, 4000, 14, 2, 64, extra=77, forced=True, rows=list(range(0, 700, 9)) + [699])


def test_noncausal(device):
    run_case(device, 4, 600, 0, 8, 8, 128, causal=False, extra=6000, forced=True, rows=list(range(0, 600, 11)) + [599])


def test_forced_off_is_the_grid(device):
    # prefill_stream = -1 with a workspace runs the grid: bitwise the output of mx_attn_prefill
    n_q, p0, nh, nkv, hd = 2048, 6144, 28, 4, 64
    _, _, _, (dq, dk, dv) = inputs(device, 5, n_q, p0 + n_q, nh, nkv, hd)
    kw = dict(n_head=nh, n_head_kv=nkv, head_dim=hd, p0=p0, want_lse=True)
    a, la = A.prefill(dq, dk, dv, **kw)
    b, lb = A.prefill(dq, dk, dv, workspace="auto", tuning=dict(prefill_stream=-1), **kw)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(la, lb)


def test_small_workspace_runs_the_grid(device):
    # a workspace too small for the stream-K slots: the grid runs (bitwise mx_attn_prefill), no error
    n_q, p0, nh, nkv, hd = 2048, 2048, 28, 4, 64
    _, _, _, (dq, dk, dv) = inputs(device, 6, n_q, p0 + n_q, nh, nkv, hd)
    kw = dict(n_head=nh, n_head_kv=nkv, head_dim=hd, p0=p0, want_lse=True)
    a, la = A.prefill(dq, dk, dv, **kw)
    b, lb = A.prefill(dq, dk, dv, workspace=A.new_workspace(1 << 20, device), **kw)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(la, lb)


def test_rope_chunks(device):
    # the fused prompt path (rope_store, then stream-K on the rotated f32 rows) over 3 chunks of 2048, against the grid
    # (whose rotated path the rope prefill tests check against the oracle): outputs within the tolerance, caches equal
    nh, nkv, hd, M = 28, 4, 128, 2048
    N = 3 * M
    rng = np.random.default_rng(7)
    qkv = torch.from_numpy(rng.standard_normal((N, (nh + 2 * nkv) * hd)).astype(np.float32) * 0.5).to(device)
    outs = []
    for ws, tun in ((None, None), ("auto", dict(prefill_stream=1))):
        kc = torch.zeros(N, nkv * hd, dtype=torch.float16, device=device)
        vc = torch.zeros_like(kc)
        out = torch.empty(N, nh * hd, dtype=torch.float32, device=device)
        for p0 in range(0, N, M):
            A.prefill_rope(qkv[p0:p0 + M], kc, vc, n_head=nh, n_head_kv=nkv, head_dim=hd, rope_mode=1,
                           rope_base=1000000.0, p0=p0, out=out[p0:p0 + M], workspace=ws, tuning=tun)
        torch.cuda.synchronize()
        outs.append((out.cpu().numpy(), kc, vc))
    np.testing.assert_allclose(outs[1][0], outs[0][0], atol=2e-3, rtol=0)
    assert torch.equal(outs[0][1], outs[1][1]) and torch.equal(outs[0][2], outs[1][2])
