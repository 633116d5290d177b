"""Randomized parity sweep of the fused entry points that take the reference's f32 q|k|v rows: mx_attn_decode_rope
(rotary embedding + cache append + decode, llama_kernels.h:552-630) and mx_attn_prefill_rope[_ws] (rope_store +
attention_prefill, llama_kernels.h:520-545, 632-769). Every case draws its shape from a seeded generator: GQA groups
of 1..16 query heads per kv head, head dims 64 and 128, the three rotation modes (adjacent, neox, none) with bases
1e4..1e6, decode batches of 1..5 sequences of 1..12000 keys, prompt chunks of 1..700 rows at offsets 0..20000 with and
without a workspace (so the decode route, the stream-K split and the grid all take rotated queries). The checks are
those of the directed suites: written key rows within one half ulp of the oracle's rotation, value rows bit for bit,
no other cache row touched, and the output against the f64 oracle. MX_FUZZ_SEEDS widens the sweep."""
import os

import numpy as np
import pytest

from test_decode_rope_gpu import run_rope
from test_prefill_rope_gpu import run_prefill_rope

pytestmark = pytest.mark.gpu

SEEDS = int(os.environ.get("MX_FUZZ_SEEDS", "10"))
GROUPS = [(1, 1), (4, 1), (7, 1), (8, 2), (14, 2), (16, 1), (20, 20), (28, 4), (32, 8), (12, 3)]
BASES = [10000.0, 500000.0, 1000000.0]


@pytest.mark.parametrize("seed", range(SEEDS))
def test_decode_rope_fuzz(device, seed):
    rng = np.random.default_rng(5000 + seed)
    nh, nkv = GROUPS[rng.integers(len(GROUPS))]
    hd = [64, 128][rng.integers(2)]
    mode = int(rng.integers(3))
    base = BASES[rng.integers(len(BASES))]
    batch = int(rng.integers(1, 6))
    hi = 12001 if rng.random() < 0.5 else 300
    lens = [int(x) for x in rng.integers(1, hi, size=batch)]
    heads = sorted({0, nh - 1, int(rng.integers(nh))})
    run_rope(device, 6000 + seed, nh, nkv, hd, lens, mode, base, check_heads=heads, poison=bool(seed % 2))


@pytest.mark.parametrize("seed", range(SEEDS))
def test_prefill_rope_fuzz(device, seed):
    rng = np.random.default_rng(7000 + seed)
    nh, nkv = GROUPS[rng.integers(len(GROUPS))]
    hd = [64, 128][rng.integers(2)]
    mode = int(rng.integers(3))
    base = BASES[rng.integers(len(BASES))]
    M = int(rng.integers(1, 701))
    p0 = int(rng.integers(3 * M, min(20 * M, 20000) + 1)) if rng.random() < 0.6 else int(rng.integers(0, 1501))
    ws = "auto" if rng.random() < 0.7 else None
    rows = sorted({0, M - 1, int(rng.integers(M)), int(rng.integers(M))})
    heads = sorted({0, nh - 1, int(rng.integers(nh))})
    run_prefill_rope(device, 8000 + seed, nh, nkv, hd, M, p0, mode, base, rows=rows, heads=heads, workspace=ws)
