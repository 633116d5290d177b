"""Randomized parity sweep of the decode and prefill entry points against the f64 oracle (the same tolerance as the
directed suites, helpers.assert_close). Every case draws its shape from a seeded generator: GQA groups of 1..16 query
heads per kv head, head dims 4..256, cache lengths 1..6000, 1..5 sequences, 1..8 query rows, causal or not, input
scales 0.25..2; prefill chunks of 1..600 rows at offsets 0..1500 with every plan; long caches (single sequences up to
40k keys, batches of about one length and ragged ones), chunks behind prefixes of 3..20x their length, and chunks with
the plan or the stream-K split forced, causal or not. MX_FUZZ_SEEDS sets the seeds of every sweep. The seed of a
failing case is in its test id, so the case reruns alone. Mirrors the reference's shape sweeps over its attention kernels
(tests/unit/test_metal_llama_decoder.cpp, tests/unit/test_backend_ggml.cpp:677-745)."""
import os

import numpy as np
import pytest
import torch

from dooms_amd import attention as A
from helpers import assert_close, normal_f16, ref_attention

pytestmark = pytest.mark.gpu

GROUPS = [(1, 1), (4, 1), (7, 1), (8, 2), (14, 2), (16, 1), (20, 20), (28, 4), (32, 8), (12, 3)]
HEAD_DIMS = [64, 128, 64, 128, 256, 32, 16]


def _seeds(default):
    return int(os.environ.get("MX_FUZZ_SEEDS", default))


@pytest.mark.parametrize("seed", range(_seeds(24)))
def test_decode_fuzz(device, seed):
    rng = np.random.default_rng(1000 + seed)
    nh, nkv = GROUPS[rng.integers(len(GROUPS))]
    hd = HEAD_DIMS[rng.integers(len(HEAD_DIMS))]
    batch = int(rng.integers(1, 6))
    n_q = int(rng.integers(1, 9)) if rng.random() < 0.3 else 1
    causal = bool(rng.random() < 0.5) and n_q > 1
    lens = [int(x) for x in rng.integers(max(n_q, 1), 6001, size=batch)]
    if rng.random() < 0.3:
        lens = [int(x) for x in rng.integers(max(n_q, 1), 140, size=batch)]
    sigma = float(rng.choice([0.25, 0.5, 1.0, 2.0]))
    kvw = nkv * hd
    q = normal_f16(rng, (batch * n_q, nh * hd), sigma)
    ks = [normal_f16(rng, (L, kvw), sigma) for L in lens]
    vs = [normal_f16(rng, (L, kvw), sigma) for L in lens]
    scale = 1.0 / np.sqrt(hd)
    out, lse = A.decode(torch.from_numpy(q).to(device), [torch.from_numpy(k).to(device) for k in ks],
                        [torch.from_numpy(v).to(device) for v in vs], lens, n_head=nh, n_head_kv=nkv, head_dim=hd,
                        n_q=n_q, causal=causal, want_lse=True)
    torch.cuda.synchronize()
    out = out.cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy()
    heads = sorted({0, nh - 1, int(rng.integers(nh))})
    cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
    for b in range(batch):
        ro, rl = ref_attention(q[b * n_q:(b + 1) * n_q], ks[b], vs[b], nh, nkv, hd, scale, p0=lens[b] - n_q,
                               causal=causal, heads=heads)
        assert_close(out[b * n_q:(b + 1) * n_q][:, cols], ro, hd,
                     f"seed {seed}: {nh}/{nkv} hd {hd} lens {lens} n_q {n_q} causal {causal} sigma {sigma}",
                     lse[b * n_q:(b + 1) * n_q][:, heads], rl)


@pytest.mark.parametrize("seed", range(_seeds(24)))
def test_prefill_fuzz(device, seed):
    rng = np.random.default_rng(2000 + seed)
    nh, nkv = GROUPS[rng.integers(len(GROUPS))]
    hd = HEAD_DIMS[rng.integers(len(HEAD_DIMS))]
    M = int(rng.integers(1, 601))
    p0 = int(rng.integers(0, 1501)) if rng.random() < 0.6 else 0
    sigma = float(rng.choice([0.25, 0.5, 1.0, 2.0]))
    plan = int(rng.choice([0, 0, 2, 4, 8]))
    ws = "auto" if rng.random() < 0.5 else None
    N = p0 + M
    q = normal_f16(rng, (M, nh * hd), sigma)
    k = normal_f16(rng, (N, nkv * hd), sigma)
    v = normal_f16(rng, (N, nkv * hd), sigma)
    scale = 1.0 / np.sqrt(hd)
    out, lse = A.prefill(torch.from_numpy(q).to(device), torch.from_numpy(k).to(device),
                         torch.from_numpy(v).to(device), n_head=nh, n_head_kv=nkv, head_dim=hd, p0=p0, scale=scale,
                         want_lse=True, workspace=ws, tuning={"prefill_plan": plan} if plan else None)
    torch.cuda.synchronize()
    rows = sorted({0, M - 1, int(rng.integers(M)), int(rng.integers(M))})
    heads = sorted({0, nh - 1, int(rng.integers(nh))})
    # the oracle on the chosen rows: prepend the cache rows before p0 as rows of a longer query block (causal offset)
    qq = np.zeros((N, nh * hd), np.float16)
    qq[p0:] = q
    ro, rl = ref_attention(qq, k, v, nh, nkv, hd, scale, causal=True, rows=[p0 + r for r in rows], heads=heads)
    cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
    got = out.cpu().numpy().astype(np.float64)[rows][:, cols]
    assert_close(got, ro, hd, f"seed {seed}: {nh}/{nkv} hd {hd} M {M} p0 {p0} plan {plan} ws {ws} sigma {sigma}",
                 lse.cpu().numpy()[rows][:, heads], rl)


@pytest.mark.parametrize("seed", range(_seeds(12)))
def test_prefill_long_prefix_fuzz(device, seed):
    # chunks behind prefixes of 3..20x their length through mx_attn_prefill_ws with the planned route: the decode route
    # for few rows, the flash kernel split by stream-K (all CUs, or fewer ranges for small launches), or its grid
    rng = np.random.default_rng(3000 + seed)
    nh, nkv = GROUPS[rng.integers(len(GROUPS))]
    hd = [64, 128][rng.integers(2)]
    M = int(rng.integers(32, 1101))
    p0 = int(rng.integers(3 * M, min(20 * M, 20000) + 1))
    sigma = float(rng.choice([0.25, 0.5, 1.0]))
    N = p0 + M
    q = normal_f16(rng, (M, nh * hd), sigma)
    k = normal_f16(rng, (N, nkv * hd), sigma)
    v = normal_f16(rng, (N, nkv * hd), sigma)
    scale = 1.0 / np.sqrt(hd)
    out, lse = A.prefill(torch.from_numpy(q).to(device), torch.from_numpy(k).to(device),
                         torch.from_numpy(v).to(device), n_head=nh, n_head_kv=nkv, head_dim=hd, p0=p0, scale=scale,
                         want_lse=True, workspace="auto")
    torch.cuda.synchronize()
    rows = sorted({0, M - 1, int(rng.integers(M)), int(rng.integers(M))})
    heads = sorted({0, nh - 1, int(rng.integers(nh))})
    ro, rl = ref_attention(q, k, v, nh, nkv, hd, scale, p0=p0, causal=True, rows=rows, heads=heads)
    cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
    got = out.cpu().numpy().astype(np.float64)[rows][:, cols]
    assert_close(got, ro, hd, f"seed {seed}: {nh}/{nkv} hd {hd} M {M} p0 {p0} sigma {sigma}",
                 lse.cpu().numpy()[rows][:, heads], rl)


@pytest.mark.parametrize("seed", range(_seeds(8)))
def test_decode_long_fuzz(device, seed):
    # long caches: one sequence of up to 40k keys (few kv heads: up to 64 splits) or batches of 4..6 of about one length
    # (the 8-split plan) or ragged; head dims 64 and 128, one query row
    rng = np.random.default_rng(4000 + seed)
    nh, nkv = GROUPS[rng.integers(len(GROUPS))]
    hd = [64, 128][rng.integers(2)]
    kind = seed % 3
    if kind == 0:
        lens = [int(rng.integers(20000, 40001))]
    elif kind == 1:
        base = int(rng.integers(4096, 9001))
        lens = [int(base * rng.uniform(1.0, 1.4)) for _ in range(int(rng.integers(4, 7)))]
    else:
        lens = [int(x) for x in rng.integers(1, 12001, size=int(rng.integers(2, 6)))]
    batch = len(lens)
    sigma = float(rng.choice([0.25, 0.5, 1.0]))
    kvw = nkv * hd
    q = normal_f16(rng, (batch, nh * hd), sigma)
    ks = [normal_f16(rng, (L, kvw), sigma) for L in lens]
    vs = [normal_f16(rng, (L, kvw), sigma) for L in lens]
    scale = 1.0 / np.sqrt(hd)
    out, lse = A.decode(torch.from_numpy(q).to(device), [torch.from_numpy(k).to(device) for k in ks],
                        [torch.from_numpy(v).to(device) for v in vs], lens, n_head=nh, n_head_kv=nkv, head_dim=hd,
                        want_lse=True)
    torch.cuda.synchronize()
    out = out.cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy()
    heads = sorted({0, nh - 1, int(rng.integers(nh))})
    cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
    for b in range(batch):
        ro, rl = ref_attention(q[b:b + 1], ks[b], vs[b], nh, nkv, hd, scale, p0=lens[b] - 1, causal=False, heads=heads)
        assert_close(out[b:b + 1][:, cols], ro, hd, f"seed {seed}: {nh}/{nkv} hd {hd} lens {lens} sigma {sigma}",
                     lse[b:b + 1][:, heads], rl)


@pytest.mark.parametrize("seed", range(_seeds(12)))
def test_prefill_forced_fuzz(device, seed):
    # chunks through mx_attn_prefill_ws with the plan or the stream-K split forced by the tuning fields, causal behind a
    # prefix or not causal over a cache of any length (every query row sees every key)
    rng = np.random.default_rng(3500 + seed)
    nh, nkv = GROUPS[rng.integers(len(GROUPS))]
    hd = [64, 128][rng.integers(2)]
    M = int(rng.integers(1, 1101))
    causal = bool(rng.random() < 0.6)
    N = (M + int(rng.integers(0, 12001))) if causal else int(rng.integers(1, 12001))
    p0 = N - M if causal else 0
    tuning = {"prefill_stream": int(rng.choice([1, 1, -1]))} if rng.random() < 0.5 else {"prefill_plan": int(rng.choice([2, 4, 8]))}
    sigma = float(rng.choice([0.25, 0.5, 1.0]))
    q = normal_f16(rng, (M, nh * hd), sigma)
    k = normal_f16(rng, (N, nkv * hd), sigma)
    v = normal_f16(rng, (N, nkv * hd), sigma)
    scale = 1.0 / np.sqrt(hd)
    what = f"seed {seed}: {nh}/{nkv} hd {hd} M {M} N {N} causal {causal} tuning {tuning} sigma {sigma}"
    print(what, flush=True)
    out, lse = A.prefill(torch.from_numpy(q).to(device), torch.from_numpy(k).to(device),
                         torch.from_numpy(v).to(device), n_head=nh, n_head_kv=nkv, head_dim=hd, p0=p0, causal=causal,
                         n_kv=N, scale=scale, want_lse=True, workspace="auto", tuning=tuning)
    torch.cuda.synchronize()
    rows = sorted({0, M - 1, int(rng.integers(M)), int(rng.integers(M))})
    heads = sorted({0, nh - 1, int(rng.integers(nh))})
    ro, rl = ref_attention(q, k, v, nh, nkv, hd, scale, p0=p0, causal=causal, rows=rows, heads=heads)
    cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
    got = out.cpu().numpy().astype(np.float64)[rows][:, cols]
    assert_close(got, ro, hd, what, lse.cpu().numpy()[rows][:, heads], rl)
