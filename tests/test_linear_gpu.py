"""Parity of mx_linear (the projections either side of the attention) with the oracle, through the C ABI.

Replaces matvec1 / matvecm (llama_kernels.h:96-126, 809-842) for M <= 8 rows and matmul / matmul_big with rms_scale
(llama_kernels.h:164-300, 309-450) for prompt chunks, and the Whisper cross-attention cache producer (matmul_big then
to_half, metal_whisper_decoder.mm:295-316). Shapes are the decoders' own: Llama-3-8B / Qwen2.5 q|k|v and attn_output,
Whisper large-v3-turbo (n_state 1280) prompt rows and the 1500-frame cross cache.

Tolerance (f32 accumulation against the oracle's double sums of the same operands), per output element with
S = sum_k |a_k w_k|: the f32-input path |y - ref| <= 1e-5 S + 1e-6; the half-operand path likewise when the inputs are
not normalized (the GPU and the oracle round x to half identically) and 2^-10 S + 1e-6 with the RMS norm (the row
scale may differ in its last f32 bit between the two reductions, which can move an operand to the neighbouring half);
f16 outputs add half an ulp of the result.
"""
import numpy as np
import pytest
import torch

from dooms_amd import attention as A
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def check(got, x, w, gamma, bias, eps, half_input, accumulate_from=None, out_f16=False, rows=None, what=""):
    rows = np.arange(x.shape[0]) if rows is None else np.asarray(rows)
    flags = (1 if gamma is not None else 0) | (4 if bias is not None else 0) | (2 if accumulate_from is not None else 0)
    xs = x[rows]
    y0 = None if accumulate_from is None else accumulate_from[rows].astype(np.float64)
    ref = O.linear_f64(xs, w, flags=flags, half_input=half_input, eps=eps, gamma=gamma, bias=bias, y0=y0)
    # S = sum_k |a_k w_k| with the oracle's operands (matvec form: x * gamma * scale)
    if gamma is not None:
        scale = 1 / np.sqrt((xs.astype(np.float64) ** 2).mean(axis=1) + eps)
        a = np.abs(xs.astype(np.float64) * gamma[None, :] * scale[:, None])
    else:
        a = np.abs(xs.astype(np.float64))
    S = a @ np.abs(w.astype(np.float64)).T
    rel = (2.0 ** -10 if (half_input and gamma is not None) else 1e-5)
    tol = rel * S + 1e-6
    g = got[rows].astype(np.float64)
    if out_f16:
        tol = tol + np.abs(ref) * 2.0 ** -11 + 2.0 ** -25
    err = np.abs(g - ref)
    assert np.all(np.isfinite(g)), what
    bad = err > tol
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} out of tolerance, max err {err.max():.3e}"


def run(device, seed, M, N, K, norm=False, bias=False, accumulate=False, out_f16=False, count=1, rows=None,
        x_pad=0, y_pad=0, eps=1e-5):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, K + x_pad), dtype=np.float32) * 2)
    ws = [(rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float16) for _ in range(count)]
    gamma = rng.uniform(0.2, 2.0, K).astype(np.float32) if norm else None
    biases = [rng.standard_normal(N).astype(np.float32) for _ in range(count)] if bias else None
    odt = np.float16 if out_f16 else np.float32
    y0 = [rng.standard_normal((M, N + y_pad)).astype(odt) for _ in range(count)]
    dx = torch.from_numpy(x).to(device)
    dws = [torch.from_numpy(w).to(device) for w in ws]
    douts = [torch.from_numpy(y.copy()).to(device) for y in y0]
    dgamma = None if gamma is None else torch.from_numpy(gamma).to(device)
    dbias = None if biases is None else [torch.from_numpy(b).to(device) for b in biases]
    xin = dx[:, :K] if x_pad == 0 else dx
    A.linear(xin, dws, out=[o[:, :N] for o in douts], gamma=dgamma, bias=dbias, eps=eps, accumulate=accumulate,
             out_f16=out_f16)
    torch.cuda.synchronize()
    half_input = M > 8
    for i in range(count):
        got = douts[i].cpu().numpy()
        check(got[:, :N], x[:, :K], ws[i], gamma, None if biases is None else biases[i], eps, half_input,
              accumulate_from=y0[i][:, :N] if accumulate else None, out_f16=out_f16, rows=rows,
              what=f"M={M} N={N} K={K} matrix {i}")
        if y_pad:  # padding columns untouched
            assert np.array_equal(got[:, N:], y0[i][:, N:])


# ---- one token (matvec1): q|k|v with the RMS norm, attn_output into the residual ----
def test_llama3_8b_qkv_decode(device):
    run(device, 1, 1, 6144, 4096, norm=True)


def test_qwen05b_qkv_decode_bias(device):
    run(device, 2, 1, 1152, 896, norm=True, bias=True)


def test_llama3_8b_attn_output_accumulate(device):
    run(device, 3, 1, 4096, 4096, accumulate=True)


# ---- up to 8 rows (matvecm): Whisper prompt rows, staged and unstaged input ----
@pytest.mark.parametrize("M", [2, 3, 5, 8])
def test_whisper_rows(device, M):
    run(device, 10 + M, M, 1280, 1280, bias=True)


def test_eight_rows_unstaged_input_with_norm(device):
    run(device, 4, 8, 1024, 4096, norm=True, bias=True)  # 8 x 4096 f32 exceeds the 64 KB staging budget


@pytest.mark.parametrize("M,N,K,norm", [(1, 256, 14336, True), (1, 4096, 14336, False), (4, 512, 8192, True),
                                         (2, 96, 2080, True)])
def test_input_staged_in_several_batches(device, M, N, K, norm):
    # input rows longer than one batch of the staging loads (a workgroup of one wave holds 4 (M = 1) or 2 (M = 2)
    # 16-byte pieces per row per thread per batch); the FFN-down shape accumulates into the residual
    run(device, 20 + M + K, M, N, K, norm=norm, accumulate=not norm)


@pytest.mark.parametrize("M,N,K,count", [(1, 4095, 4096, 1), (1, 1281, 1280, 3), (2, 1001, 896, 2), (8, 777, 512, 1),
                                          (1, 3, 64, 1), (3, 513, 256, 2)])
def test_gemv_odd_rows(device, M, N, K, count):
    # odd output widths: the last 2- or 4-row group of a wave reads a clamped row and stores only the rows it owns (the
    # output rows padded to a multiple of 4 columns, as the library requires; the padding stays untouched)
    run(device, 40 + M + N, M, N, K, bias=True, accumulate=True, count=count, y_pad=-N % 4)


# ---- prompt chunks (matmul): the MFMA GEMM ----
def test_qwen05b_prompt_qkv(device):
    run(device, 5, 512, 1152, 896, norm=True, bias=True, rows=list(range(0, 512, 5)) + [511])


def test_gemm_ragged_edges(device):
    run(device, 6, 131, 200, 96, bias=True, accumulate=True)


@pytest.mark.parametrize("M,N,K", [(9, 64, 32), (33, 132, 160), (200, 256, 192), (129, 96, 320)])
def test_gemm_step_counts(device, M, N, K):
    """K steps of 64 (the last one half zero-padded when K is an odd multiple of 32), odd and even step counts
    (the GEMM's main loop runs steps in pairs and finishes an odd count alone), the smallest GEMM row count."""
    run(device, 20 + K, M, N, K, norm=True, bias=True)


def test_gemm_big_tiles_ragged(device):
    """A product with enough 256 x 256 tiles for the large-tile GEMM: M and N not multiples of 256 (rows and
    columns past them repeat the last one and are never stored), 5 steps of 32 columns, with the RMS normalization,
    bias and accumulation; rows sampled across the tiles and at both edges."""
    run(device, 10, 1300, 8300, 160, norm=True, bias=True, accumulate=True,
        rows=[0, 1, 255, 256, 511, 700, 1023, 1024, 1279, 1280, 1299])


def test_gemm_mid_tiles_ragged(device):
    """Enough 256 x 128 tiles (but too few 256 x 256 ones) for the 256 x 128 GEMM: ragged M and N, 3 steps of 32
    columns, f16 output with bias."""
    run(device, 11, 1900, 3896, 96, bias=True, out_f16=True, rows=[0, 1, 255, 256, 1023, 1536, 1791, 1792, 1899])


def test_gemm_w192_tiles_ragged(device):
    """A product that takes the 256 x 192 tiles (8 waves of 64 x 96 columns, the B tile's 12 load blocks spread over
    16 loads): ragged M and N, 3 steps of 32 columns, accumulation."""
    run(device, 12, 1900, 5700, 96, accumulate=True, rows=[0, 1, 255, 256, 1023, 1536, 1791, 1792, 1899])


@pytest.mark.parametrize("K", [64, 192, 320])
@pytest.mark.parametrize("M,N,opts", [
    (1300, 8300, dict(norm=True, bias=True, accumulate=True)),  # 256 x 256 tiles
    (1900, 3896, dict(bias=True, out_f16=True)),                # 256 x 128 tiles
    (1900, 5700, dict(accumulate=True)),                        # 256 x 192 tiles
])
def test_gemm_tiles_ragged_k64_steps(device, M, N, opts, K):
    """The same ragged products with K a multiple of 64, which the tiled GEMMs walk in steps of 64 columns through
    two LDS buffers: one step, three and five (the buffer ring wrapping at an odd count)."""
    run(device, 13 + K, M, N, K, rows=[0, 1, 255, 256, 1023, 1024, M - 2, M - 1], **opts)


def test_gemm_llama3_attn_output_chunk(device):
    run(device, 7, 300, 4096, 4096, accumulate=True, rows=[0, 1, 127, 128, 255, 299])


def test_gemm_padded_strides(device):
    run(device, 8, 40, 72, 64, norm=True, x_pad=12, y_pad=8)


def test_gemv_padded_strides_f16(device):
    run(device, 9, 3, 72, 64, norm=True, out_f16=True, x_pad=4, y_pad=8)


# ---- the Whisper cross-attention cache: K and V of 4 layers in one launch, f16 rows ----
def test_whisper_cross_kv_cache(device):
    rng = np.random.default_rng(12)
    A_, d, L = 1500, 1280, 4
    x = rng.standard_normal((A_, d), dtype=np.float32)
    ws = [(rng.standard_normal((d, d), dtype=np.float32) / np.sqrt(d)).astype(np.float16) for _ in range(2 * L)]
    biases = [None if i % 2 == 0 else rng.standard_normal(d).astype(np.float32) for i in range(2 * L)]  # K: no bias
    dev = lambda a: torch.from_numpy(a).to(device)
    outs = A.linear(dev(x), [dev(w) for w in ws], bias=[None if b is None else dev(b) for b in biases],
                    out_f16=True)
    torch.cuda.synchronize()
    rows = [0, 1, 63, 64, 127, 128, 700, 1407, 1408, 1499]
    for i in range(2 * L):
        got = outs[i].cpu().numpy()
        assert got.dtype == np.float16
        check(got, x, ws[i], None, biases[i], 1e-5, True, out_f16=True, rows=rows, what=f"cross matrix {i}")


def test_linear_rejects_mismatched_shapes(device):
    x = torch.zeros(2, 64, device=device)
    with pytest.raises(ValueError):
        A.linear(x, [torch.zeros(8, 64, dtype=torch.float16, device=device),
                     torch.zeros(16, 64, dtype=torch.float16, device=device)])
