"""Randomized parity sweep of mx_linear (matvec1 / matvecm / matmul / matmul_big with rms_scale, llama_kernels.h:96-126,
164-450, 809-842) and mx_self_attention (the IR's SelfAttention op, src/ir/op.h:31-32) against the f64 oracle, with the
tolerances of the directed suites (test_linear_gpu.check, helpers.assert_close). Linear: 1..700 input rows (the GEMV up
to 8, the MFMA GEMM tiles beyond), 1..3000 outputs, 32..4096 inputs in steps of 32, 1..4 matrices, the RMS norm, bias,
accumulation and f16 outputs drawn at random, odd widths padded to the stride rule. Self-attention: 1..3 sequences of
1..700 tokens, 1..16 heads of head dim 4..128 (odd ones included), f32 / f16 / bf16 rows. MX_FUZZ_SEEDS widens the
sweep."""
import os

import numpy as np
import pytest

import test_linear_gpu as L
import test_self_attention_gpu as S

pytestmark = pytest.mark.gpu

SEEDS = int(os.environ.get("MX_FUZZ_SEEDS", "10"))


@pytest.mark.parametrize("seed", range(SEEDS))
def test_linear_fuzz(device, seed):
    rng = np.random.default_rng(9000 + seed)
    M = int(rng.integers(1, 9)) if rng.random() < 0.5 else int(rng.integers(9, 701))
    N = int(rng.integers(1, 3001))
    K = 32 * int(rng.integers(1, 129))
    out_f16 = bool(rng.random() < 0.3)
    y_pad = -N % (8 if out_f16 else 4)
    rows = None if M <= 64 else sorted({0, M - 1, *(int(r) for r in rng.integers(0, M, 14))})
    print(f"linear seed {seed}: M={M} N={N} K={K} f16 out {out_f16}", flush=True)
    L.run(device, 9500 + seed, M, N, K, norm=bool(rng.random() < 0.5), bias=bool(rng.random() < 0.3),
          accumulate=bool(rng.random() < 0.3), out_f16=out_f16, count=int(rng.integers(1, 5)), rows=rows,
          x_pad=4 * int(rng.integers(0, 3)), y_pad=y_pad)


@pytest.mark.parametrize("seed", range(SEEDS))
def test_self_attention_fuzz(seed):
    rng = np.random.default_rng(9800 + seed)
    B = int(rng.integers(1, 4))
    N = int(rng.integers(1, 701)) if rng.random() < 0.7 else int(rng.integers(1, 40))
    H = int(rng.integers(1, 17))
    D = int(rng.choice([4, 6, 8, 16, 24, 32, 48, 64, 80, 96, 128]))
    dtype = ["f32", "f16", "bf16"][rng.integers(3)]
    S.run(B, N, H, D, dtype, seed=9900 + seed)
