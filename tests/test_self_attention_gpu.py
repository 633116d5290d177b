"""Parity of mx_self_attention (the IR's SelfAttention op, src/ir/op.h:31-32) with the f64 oracle, through the C ABI.

Cases are the reference's own (kAttnCases, tests/unit/test_backend_ggml.cpp:677-681: odd head dims 4, 6, 8 and 16, a
one-token sequence, batch 2, the ViT-H shape of 210 tokens x 16 heads of 80), in f32, f16 and bf16, plus larger
shapes that take every path: f16 rows read in place (head_dim 64/128), f32 rows with the f16 key/value copy, and padded
operands. Inputs are U(-1, 1) like the reference's rnd().

Tolerance: against the f64 oracle on the operands the kernel multiplies (the inputs rounded to half), the build's bound
|got - ref| <= 2e-3 + 1e-2 |ref| elementwise (tests/helpers.py; it also covers the bf16 output's rounding, 2^-9
relative); and for scales up to head_dim^-0.5, against the oracle on the exact inputs, the reference's GPU bound max abs
error <= 3e-3 (test_backend_ggml.cpp:694, Metal's flash attention rounds Q/K/V to half as this kernel does). Larger
scales magnify the half rounding of q and k in the scores, so only the first comparison applies to them.
"""
import numpy as np
import pytest
import torch

from dooms_amd import _lib
from dooms_amd import attention as A
from oracle import oracle as O
from helpers import assert_close

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
REF_CASES = [(1, 5, 2, 4), (2, 7, 3, 8), (1, 1, 1, 16), (1, 17, 4, 64), (1, 9, 2, 6), (1, 210, 16, 80)]


def run(B, N, H, D, dtype, scale=None, seed=0):
    rng = np.random.default_rng(seed or 700 + N)
    E = H * D
    x = torch.from_numpy(rng.uniform(-1, 1, (B, N, 3 * E)).astype(np.float32)).to(DT[dtype])
    exact = x.float().numpy()  # the values the GPU receives, exactly
    scale = D ** -0.5 if scale is None else scale
    print(f"self_attention B={B} N={N} H={H} D={D} {dtype} scale={scale}", flush=True)
    y = A.self_attention(x.cuda(), heads=H, scale=scale)
    torch.cuda.synchronize()
    assert y.dtype == DT[dtype] and tuple(y.shape) == (B, N, E)
    # the kernel's operands are the inputs rounded to half (the reference's GPU path rounds them too)
    ref = O.self_attention_f64(exact.astype(np.float16).astype(np.float64), H, scale)
    got = y.float().cpu().numpy()
    assert_close(got.reshape(B * N, E), ref.reshape(B * N, E), D, what=f"B={B} N={N} H={H} D={D} {dtype}")
    if abs(scale) <= D ** -0.5:  # and the reference's own bound against the exact inputs
        err = np.abs(got - O.self_attention_f64(exact, H, scale)).max()
        assert err <= 3e-3, err
    return got, ref


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("B,N,H,D", REF_CASES)
def test_reference_cases(B, N, H, D, dtype):
    run(B, N, H, D, dtype)


@pytest.mark.parametrize("B,N,H,D,dtype", [
    (2, 1000, 8, 64, "f16"),     # in place, several query tiles, batch along the grid
    (1, 577, 12, 64, "f32"),     # ViT-B/16 at 384 px: f32 rows, f16 key/value copy
    (2, 300, 4, 128, "f32"),
    (3, 129, 6, 128, "f16"),
    (1, 257, 16, 80, "bf16"),    # padded operands
    (2, 513, 5, 96, "f32"),
    (1, 2048, 16, 64, "f16"),    # 8-wave workgroups
])
def test_larger_shapes(B, N, H, D, dtype):
    run(B, N, H, D, dtype)


@pytest.mark.parametrize("scale", [0.0, 0.1, 0.5, 3.0, -0.5])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_scale_semantics(scale, dtype):
    """op_self_attention_scale_semantics (test_backend_ggml.cpp:712-735): scale 0 is uniform attention, every output row
    the mean of v over the tokens; negative scales too."""
    got, ref = run(1, 6, 2, 8, dtype, scale=scale, seed=710)
    got2, _ = run(1, 70, 2, 64, dtype, scale=scale, seed=711)
    if scale == 0.0:
        np.testing.assert_allclose(got[0], np.broadcast_to(ref[0].mean(axis=0), got[0].shape), atol=3e-3)


def test_batch_elements_are_independent():
    """Element b of a batch equals the same rows run alone (the grid's batch offsets)."""
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.uniform(-1, 1, (3, 200, 3 * 256)).astype(np.float16)).cuda()
    y = A.self_attention(x, heads=4)
    for b in range(3):
        yb = A.self_attention(x[b:b + 1].contiguous(), heads=4)
        assert torch.equal(y[b:b + 1], yb)


def test_dtype_paths_agree():
    """f32 rows (in-kernel f32 query, f16 keys/values) and the same rows given as f16 differ only by the query rounding."""
    rng = np.random.default_rng(6)
    x32 = torch.from_numpy(rng.uniform(-1, 1, (1, 333, 3 * 512)).astype(np.float16).astype(np.float32)).cuda()
    y32 = A.self_attention(x32, heads=8)
    y16 = A.self_attention(x32.half(), heads=8)
    assert (y32 - y16.float()).abs().max().item() <= 2e-3


def test_errors_leave_output_untouched():
    x = torch.zeros(1, 4, 3 * 24, device="cuda", dtype=torch.float32)
    with pytest.raises(_lib.MxAttnError) as e:
        A.self_attention(x, heads=5)
    assert e.value.code == _lib.INVALID_ARGUMENT


# the batched launch under every prefill workgroup plan (the batch runs along the grid's second dimension)
@pytest.mark.parametrize("plan", [2, 4, 8])
@pytest.mark.parametrize("B,N,H,D,dtype", [(1, 210, 16, 80, "f32"), (3, 300, 4, 64, "f16"), (2, 400, 2, 128, "bf16")])
def test_workgroup_plans(plan, B, N, H, D, dtype):
    with A.tuning(prefill_plan=plan):
        run(B, N, H, D, dtype)
