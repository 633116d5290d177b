"""Parity of mx_attn_prefill (causal GQA flash attention, MFMA) with the f64 oracle, through the C ABI.

Reference: attention_prefill<64|128> (llama_kernels.h:632-769) as dispatched by MetalLlamaDecoder::Impl::attention
(metal_llama_decoder.mm:284-296), and the chunked prompt loop against the growing cache (metal_llama_decoder.mm:703-723).
Reference tests mirrored: flash prefill on a 45-token prompt in chunks of 20 (test_metal_llama_decoder.cpp:497-532),
chunk-size invariance, non-causal MHA (test_backend_ggml.cpp:677-745).
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from dooms_amd import _lib
from dooms_amd import attention as A
from helpers import assert_close, normal_f16, ref_attention
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def make(device, seed, n_q_total, n_head, n_head_kv, hd, sigma=1.0, kv_pad=0, q_pad=0):
    rng = np.random.default_rng(seed)
    q = normal_f16(rng, (n_q_total, n_head * hd + q_pad), sigma)
    k = normal_f16(rng, (n_q_total, n_head_kv * hd + kv_pad), sigma)
    v = normal_f16(rng, (n_q_total, n_head_kv * hd + kv_pad), sigma)
    return q, k, v, [torch.from_numpy(a).to(device) for a in (q, k, v)]


def check_prefill(device, seed, N, n_head, n_head_kv, hd, rows=None, heads=None, causal=True, sigma=1.0, scale=None,
                  kv_pad=0, q_pad=0, chunk=None, workspace=None):
    q, k, v, (dq, dk, dv) = make(device, seed, N, n_head, n_head_kv, hd, sigma, kv_pad, q_pad)
    scale = 1.0 / np.sqrt(hd) if scale is None else scale
    if chunk is None:
        out, lse = A.prefill(dq, dk, dv, n_head=n_head, n_head_kv=n_head_kv, head_dim=hd, causal=causal,
                             scale=scale, want_lse=True)
    else:  # chunks at p0 = 0, chunk, 2 chunk, ... against the growing cache
        out = torch.empty(N, n_head * hd, dtype=torch.float16, device=device)
        lse = torch.empty(N, n_head, dtype=torch.float32, device=device)
        for p0 in range(0, N, chunk):
            m = min(chunk, N - p0)
            A.prefill(dq[p0:p0 + m], dk[:p0 + m], dv[:p0 + m], n_head=n_head, n_head_kv=n_head_kv, head_dim=hd,
                      p0=p0, scale=scale, out=out[p0:p0 + m], lse=lse[p0:p0 + m], workspace=workspace)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    gl = lse.cpu().numpy()
    rows = np.arange(N) if rows is None else np.asarray(rows)
    heads = np.arange(n_head) if heads is None else np.asarray(heads)
    ro, rl = ref_attention(q, k, v, n_head, n_head_kv, hd, scale, causal=causal, rows=rows, heads=heads)
    cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
    assert_close(got[rows][:, cols], ro, hd, f"N={N}", gl[rows][:, heads], rl)
    return got, gl


def test_tiny_gqa(device):
    check_prefill(device, 1, 45, 4, 2, 64)


def test_tiny_gqa_chunks_of_20(device):
    # test_metal_llama_decoder.cpp:497-532: a 45-token prompt through the flash kernel in chunks of 20
    check_prefill(device, 1, 45, 4, 2, 64, chunk=20)


@pytest.mark.parametrize("N", [1, 2, 31, 32, 63, 64, 65, 127, 128, 129, 200, 257])
def test_ragged_lengths(device, N):
    check_prefill(device, 100 + N, N, 4, 1, 128)


# cfg2: Qwen2.5-0.5B prefill of a 512-token prompt
def test_qwen05b_prefill_512(device):
    check_prefill(device, 2, 512, 14, 2, 64)


@pytest.mark.parametrize("chunk", [20, 128, 200, 512])
def test_chunked_equals_oracle(device, chunk):
    check_prefill(device, 3, 700, 14, 2, 64, rows=list(range(0, 700, 7)) + [699], chunk=chunk)


def test_noncausal_mha(device):
    # the IR SelfAttention shape class (non-causal MHA, test_backend_ggml.cpp:680)
    check_prefill(device, 4, 210, 16, 16, 64, causal=False)


@pytest.mark.parametrize("scale", [0.0, 0.1, 3.0])
def test_scale_semantics(device, scale):
    check_prefill(device, 5, 150, 4, 2, 64, scale=scale)


def test_padded_strides(device):
    # q and caches inside wider rows (a fused q|k|v buffer, say)
    check_prefill(device, 6, 300, 8, 2, 128, kv_pad=256, q_pad=512)


# cfg5 shape class: Qwen2.5-7B (28q/4kv, hd 128), sigma 0.5, in 2048-query chunks; reduced length here, full 32k below
def test_qwen7b_chunked_4096(device):
    rows = [0, 1, 2047, 2048, 2049, 3000, 4095]
    check_prefill(device, 7, 4096, 28, 4, 128, rows=rows, sigma=0.5, chunk=2048)


def test_qwen7b_32k_chunked_equals_one_shot(device):
    """cfg5 at full size: 32768 causal tokens in 16 chunks of 2048 against the growing cache.

    Size-independent properties: chunked == one-shot (bitwise: the kernel visits the same key blocks for every row
    when chunk boundaries are multiples of its 128-row tile), and sampled rows against the f64 oracle.
    """
    N, nh, nkv, hd = 32768, 28, 4, 128
    rng = np.random.default_rng(5)
    q = normal_f16(rng, (N, nh * hd), 0.5)
    k = normal_f16(rng, (N, nkv * hd), 0.5)
    v = normal_f16(rng, (N, nkv * hd), 0.5)
    dq, dk, dv = (torch.from_numpy(a).to(device) for a in (q, k, v))
    one, lse1 = A.prefill(dq, dk, dv, n_head=nh, n_head_kv=nkv, head_dim=hd, want_lse=True)
    out = torch.empty_like(one)
    lse = torch.empty_like(lse1)
    for p0 in range(0, N, 2048):
        A.prefill(dq[p0:p0 + 2048], dk[:p0 + 2048], dv[:p0 + 2048], n_head=nh, n_head_kv=nkv, head_dim=hd, p0=p0,
                  out=out[p0:p0 + 2048], lse=lse[p0:p0 + 2048])
    torch.cuda.synchronize()
    assert torch.equal(one, out)
    assert torch.equal(lse1, lse)
    # every head of rows in every chunk: the chunk's first and last rows, a 256-row workgroup tile's first and last,
    # and one more, against the f64 oracle (all heads of a row in one oracle call)
    rows = sorted({r for p0 in range(0, N, 2048) for r in (p0, p0 + 255, p0 + 256, p0 + 2047)})
    got = out.cpu().numpy().astype(np.float64)
    gl = lse.cpu().numpy()
    oracle_row = lambda t: O.attention_f64(q[t:t + 1], k[:t + 1], v[:t + 1], nh, nkv, hd, 1.0 / np.sqrt(hd), p0=t,
                                           causal=True)
    with ThreadPoolExecutor(max_workers=8) as ex:  # the C oracle runs outside the GIL
        refs = list(ex.map(oracle_row, rows))
    for t, (ro, rl) in zip(rows, refs):
        assert_close(got[t:t + 1], ro, hd, f"32k row {t}", gl[t:t + 1], rl)


def test_one_row_per_key_closed_form(device):
    # one key: O = v0 exactly (up to f16 rounding of v0 itself)
    rng = np.random.default_rng(8)
    dq, dk, dv = (torch.from_numpy(normal_f16(rng, (1, 128))).to(device) for _ in range(3))
    out, lse = A.prefill(dq, dk, dv, n_head=1, n_head_kv=1, head_dim=128, want_lse=True)
    assert torch.equal(out, dv)


def test_equal_keys_mean_of_v(device):
    rng = np.random.default_rng(9)
    N, hd = 300, 64
    q = torch.from_numpy(normal_f16(rng, (N, hd))).to(device)
    k = torch.from_numpy(np.tile(normal_f16(rng, (1, hd)), (N, 1))).to(device)
    vn = normal_f16(rng, (N, hd))
    out, _ = A.prefill(q, k, torch.from_numpy(vn).to(device), n_head=1, n_head_kv=1, head_dim=hd)
    cm = np.cumsum(vn.astype(np.float64), axis=0) / np.arange(1, N + 1)[:, None]
    np.testing.assert_allclose(out.cpu().numpy().astype(np.float64), cm, atol=2e-3, rtol=1e-2)


# every workgroup plan (8 or 4 waves of 32-row tiles, or 4 waves over two 32-row tiles each split over two key halves)
# on the same problems: chunk offsets, non-causal, zero/negative scales, ragged ends, both head dims
@pytest.mark.parametrize("plan", [2, 4, 8])
@pytest.mark.parametrize("case", ["gqa_hd128_chunks", "mha_hd64_noncausal", "neg_scale", "ragged_257", "one_block"])
def test_workgroup_plans(device, plan, case):
    with A.tuning(prefill_plan=plan):
        if case == "gqa_hd128_chunks":
            check_prefill(device, 200, 900, 8, 2, 128, rows=list(range(0, 900, 5)) + [899], chunk=300)
        elif case == "mha_hd64_noncausal":
            check_prefill(device, 201, 333, 6, 6, 64, causal=False)
        elif case == "neg_scale":
            check_prefill(device, 202, 400, 4, 2, 64, scale=-0.3)
        elif case == "ragged_257":
            check_prefill(device, 203, 257, 4, 1, 128)
        else:
            check_prefill(device, 204, 60, 4, 2, 64)


# mx_attn_prefill_ws: chunks of few rows on the split-KV decode kernel (n_q x group <= 512), larger ones on the flash
# kernel; the last chunk of each prompt is short, so every case below takes both routes
@pytest.mark.parametrize("N,chunk,n_head,n_head_kv,hd", [(1000, 17, 28, 4, 128), (700, 64, 14, 2, 64),
                                                         (3000, 2000, 32, 8, 128), (300, 1, 8, 8, 64)])
def test_prefill_ws_routes(device, N, chunk, n_head, n_head_kv, hd):
    rows = sorted(set(list(range(0, N, max(1, N // 60))) + [N - 1, N - 2, chunk - 1, chunk]))
    rows = [r for r in rows if r < N]
    check_prefill(device, 400 + N, N, n_head, n_head_kv, hd, rows=rows, chunk=chunk, workspace="auto")


@pytest.mark.parametrize("M", [16, 48, 64, 128, 200])
def test_prefill_ws_long_context(device, M):
    # the last M prompt rows at the end of a 131072-token context (Qwen2.5-7B shape): 16 and 48 rows take the split-KV
    # route, 64 and 128 rows (within its packed-row bound) the flash kernel split by stream-K over the CUs, 200 rows
    # (1400 packed rows per kv head) the flash kernel as well
    rng = np.random.default_rng(420 + M)
    L, hd, heads = 131072, 128, [0, 6, 7, 27]
    q = torch.from_numpy(normal_f16(rng, (M, 28 * hd))).to(device)
    kn, vn = normal_f16(rng, (L, 4 * hd)), normal_f16(rng, (L, 4 * hd))
    k, v = torch.from_numpy(kn).to(device), torch.from_numpy(vn).to(device)
    out, lse = A.prefill(q, k, v, n_head=28, n_head_kv=4, head_dim=hd, p0=L - M, want_lse=True, workspace="auto")
    torch.cuda.synchronize()
    rows = [0, M // 2, M - 1]
    ro, rl = ref_attention(q.cpu().numpy(), kn, vn, 28, 4, hd, 1 / np.sqrt(hd), p0=L - M, rows=rows, heads=heads)
    cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
    assert_close(out.cpu().numpy().astype(np.float64)[rows][:, cols], ro, hd, f"M={M}",
                 lse.cpu().numpy()[rows][:, heads], rl)


@pytest.mark.parametrize("M", [64, 128])
def test_prefill_ws_long_context_hd64(device, M):
    # Qwen2.5-0.5B shape (14 q / 2 kv heads of 64), the last M rows of a 32768-token context: 64 rows on the split-KV
    # route, 128 rows on the flash kernel split by stream-K
    rng = np.random.default_rng(440 + M)
    L, hd, heads = 32768, 64, [0, 6, 7, 13]
    q = torch.from_numpy(normal_f16(rng, (M, 14 * hd))).to(device)
    kn, vn = normal_f16(rng, (L, 2 * hd)), normal_f16(rng, (L, 2 * hd))
    k, v = torch.from_numpy(kn).to(device), torch.from_numpy(vn).to(device)
    out, lse = A.prefill(q, k, v, n_head=14, n_head_kv=2, head_dim=hd, p0=L - M, want_lse=True, workspace="auto")
    torch.cuda.synchronize()
    rows = [0, M // 2, M - 1]
    ro, rl = ref_attention(q.cpu().numpy(), kn, vn, 14, 2, hd, 1 / np.sqrt(hd), p0=L - M, rows=rows, heads=heads)
    cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
    assert_close(out.cpu().numpy().astype(np.float64)[rows][:, cols], ro, hd, f"M={M}",
                 lse.cpu().numpy()[rows][:, heads], rl)


def test_prefill_ws_short_workspace_keeps_route(device):
    # 128 rows at 30k keys would take the stream-K flash kernel; with a workspace sized for the decode route only (no
    # room for the stream-K slots) the chunk stays on the route, with the same results
    rng = np.random.default_rng(450)
    M, p0, hd, heads = 128, 30000, 128, [0, 6, 7, 27]
    L = p0 + M
    q = torch.from_numpy(normal_f16(rng, (M, 28 * hd))).to(device)
    kn, vn = normal_f16(rng, (L, 4 * hd)), normal_f16(rng, (L, 4 * hd))
    k, v = torch.from_numpy(kn).to(device), torch.from_numpy(vn).to(device)
    d128 = _lib.make_desc(28, 4, hd, M, 28 * hd, 4 * hd, 28 * hd, 1 / np.sqrt(hd), p0=p0, causal=1)
    small = _lib.decode_workspace_bytes(d128, 1, L)  # the route's own size for this chunk
    assert 0 < small < _lib.prefill_workspace_bytes(d128)
    ws = A.new_workspace(small, device)
    out, lse = A.prefill(q, k, v, n_head=28, n_head_kv=4, head_dim=hd, p0=p0, want_lse=True, workspace=ws)
    full, lfull = A.prefill(q, k, v, n_head=28, n_head_kv=4, head_dim=hd, p0=p0, want_lse=True, workspace="auto")
    torch.cuda.synchronize()
    rows = [0, 64, M - 1]
    ro, rl = ref_attention(q.cpu().numpy(), kn, vn, 28, 4, hd, 1 / np.sqrt(hd), p0=p0, rows=rows, heads=heads)
    cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
    for o, l, what in ((out, lse, "route"), (full, lfull, "stream-K")):
        assert_close(o.cpu().numpy().astype(np.float64)[rows][:, cols], ro, hd, what, l.cpu().numpy()[rows][:, heads], rl)


def test_prefill_ws_noncausal_and_extra_keys(device):
    # non-causal rows over n_kv keys, and a causal chunk with cache rows past its own (masked, not read)
    rng = np.random.default_rng(410)
    L, M, hd = 5000, 12, 128
    q = torch.from_numpy(normal_f16(rng, (M, 28 * hd))).to(device)
    k = torch.from_numpy(normal_f16(rng, (L, 4 * hd))).to(device)
    v = torch.from_numpy(normal_f16(rng, (L, 4 * hd))).to(device)
    for causal, p0, n_kv in [(False, 0, L), (True, 3000, L)]:
        a, la = A.prefill(q, k, v, n_head=28, n_head_kv=4, head_dim=hd, p0=p0, n_kv=n_kv, causal=causal,
                          want_lse=True, workspace="auto")
        b, lb = A.prefill(q, k, v, n_head=28, n_head_kv=4, head_dim=hd, p0=p0, n_kv=n_kv, causal=causal,
                          want_lse=True)
        torch.cuda.synchronize()
        ro, rl = ref_attention(q.cpu().numpy(), k.cpu().numpy()[:n_kv], v.cpu().numpy()[:n_kv], 28, 4, hd,
                               1 / np.sqrt(hd), p0=p0, causal=causal, heads=[0, 6, 7, 27])
        cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in [0, 6, 7, 27]])
        for out, lse in ((a, la), (b, lb)):
            assert_close(out.cpu().numpy().astype(np.float64)[:, cols], ro, hd, f"causal={causal}",
                         lse.cpu().numpy()[:, [0, 6, 7, 27]], rl)
