"""Parity of mx_attn_decode (split-KV decode + LSE merge) with the f64 oracle, through the C ABI.

Covers the reference's decode dispatches: the per-query `attention` kernel (short decode, Whisper self-attention,
llama_kernels.h:552-630), `attention_split` + `attention_combine` (long decode and Whisper cross-attention,
llama_kernels.h:856-929), and the Whisper prompt rows (metal_whisper_decoder.mm:182-203: causal rows appended at the end
of the cache). Shapes are the BASELINE configs: Qwen2.5-0.5B (14q/2kv, hd 64), Llama-3-8B (32q/8kv, hd 128), Whisper
large-v3-turbo (20 heads MHA, hd 64, 1500 encoder frames).
"""
import os

import numpy as np
import pytest
import torch

from dooms_amd import attention as A
from helpers import assert_close, normal_f16, ref_attention

pytestmark = pytest.mark.gpu


def run_decode(device, seed, n_head, n_head_kv, hd, kv_lens, n_q=1, causal=False, shared_cache=False, sigma=1.0,
               scale=None, kv_pad=0, check_seqs=None, check_heads=None):
    rng = np.random.default_rng(seed)
    batch = len(kv_lens)
    kvw = n_head_kv * hd + kv_pad
    q = normal_f16(rng, (batch * n_q, n_head * hd), sigma)
    caches = []
    for b in range(batch):
        if shared_cache and b > 0:
            caches.append(caches[0])
            continue
        caches.append((normal_f16(rng, (kv_lens[b], kvw), sigma), normal_f16(rng, (kv_lens[b], kvw), sigma)))
    scale = 1.0 / np.sqrt(hd) if scale is None else scale
    qd = torch.from_numpy(q).to(device)
    dk = [torch.from_numpy(k).to(device) for k, _ in caches]
    dv = [torch.from_numpy(v).to(device) for _, v in caches]
    out, lse = A.decode(qd, dk, dv, list(kv_lens), n_head=n_head, n_head_kv=n_head_kv, head_dim=hd, n_q=n_q,
                        causal=causal, scale=scale, want_lse=True)
    torch.cuda.synchronize()
    out = out.cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy()
    seqs = range(batch) if check_seqs is None else check_seqs
    for b in seqs:
        k, v = caches[b]
        L = kv_lens[b]
        ro, rl = ref_attention(q[b * n_q:(b + 1) * n_q], k, v, n_head, n_head_kv, hd, scale, p0=L - n_q,
                               causal=causal, heads=check_heads)
        heads = np.arange(n_head) if check_heads is None else np.asarray(check_heads)
        cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
        assert_close(out[b * n_q:(b + 1) * n_q][:, cols], ro, hd, f"seq {b} L={L}",
                     lse[b * n_q:(b + 1) * n_q][:, heads], rl)
    return out, lse


# cfg1: Qwen2.5-0.5B decode, 512 prior tokens + the new one
def test_qwen05b_decode_513(device):
    run_decode(device, 1, 14, 2, 64, [513])


@pytest.mark.parametrize("L", [1, 7, 31, 32, 33, 127, 128, 129, 511, 512, 1000])
def test_small_lengths_gqa7(device, L):
    run_decode(device, 10 + L, 14, 2, 64, [L])


# cfg3: Llama-3-8B decode, batch 1 at 8192 (north-star shape), and batches 4/16 with lengths U[1024, 8192]
def test_llama3_8b_decode_8192(device):
    run_decode(device, 3, 32, 8, 128, [8192])  # every head


@pytest.mark.parametrize("n_head,n_head_kv,n_q,causal", [(32, 8, 16, True), (16, 16, 1, False)])
def test_one_sequence_heads_per_xcd(device, n_head, n_head_kv, n_q, causal):
    # one sequence with a multiple of 8 kv heads: kv head g's splits run on XCD g % 8; 16 causal rows make 4 row tiles
    # per kv head, 16 kv heads two heads per XCD (8192 keys: 32 splits of 256 keys)
    run_decode(device, 77 + n_q, n_head, n_head_kv, 128, [8192], n_q=n_q, causal=causal)


@pytest.mark.parametrize("hd,n_head,L", [(64, 16, 3000), (256, 16, 8192), (128, 64, 5000)])
def test_one_sequence_heads_per_xcd_head_dims(device, hd, n_head, L):
    # the XCD-mapped grid at the other head dims (the per-pair publish of head dims 64 and 256, the 8-row tiles of a
    # 64-head model): partials published into the XCD's L2 and counted per XCD
    run_decode(device, 90 + hd, n_head, 8, hd, [L], check_heads=[0, 5, n_head - 1])
    run_decode_f32(device, 91 + hd, n_head, 8, hd, [L])


def test_llama3_8b_decode_128k(device):
    # a 131072-token context: 32 splits of 4096 keys per kv head, each wave walking 16 blocks before the merge
    run_decode(device, 76, 32, 8, 128, [131072], check_heads=[0, 9, 31])


@pytest.mark.parametrize("n_head,n_head_kv,hd,lens", [
    (28, 4, 128, [6841, 1638, 2310, 2721]),          # Qwen2.5-7B batch 4
    (28, 4, 128, [3000, 129, 4097]),                 # an odd batch
    (14, 2, 64, [1024, 77, 3000, 513, 2048, 1, 700, 4096]),  # Qwen2.5-0.5B batch 8
    (8, 1, 128, [5000, 300, 1000, 64, 2000, 33, 4000, 129])])  # one kv head
def test_batched_few_kv_heads(device, n_head, n_head_kv, hd, lens):
    # ragged batches of sequences with fewer than 8 kv heads, every sequence and head checked
    run_decode(device, 60 + len(lens) + n_head_kv, n_head, n_head_kv, hd, lens)


@pytest.mark.parametrize("L", [32768, 131072])
def test_qwen7b_decode_64_splits(device, L):
    # 4 kv heads at 32k+ keys: up to 64 splits of the sequence (the 32-split grid would leave CUs idle), merged by the
    # last of them
    run_decode(device, 77, 28, 4, 128, [L], check_heads=[0, 13, 27])
    if L == 32768:
        run_decode_f32(device, 78, 28, 4, 128, [L], check_heads=[0, 13, 27])


@pytest.mark.parametrize("batch", [4, 16])
def test_llama3_8b_decode_batched(device, batch):
    # every head of every sequence against the oracle (a per-split or per-XCD indexing slip cannot hide in an
    # unchecked head)
    lens = list(np.random.default_rng(300 + batch).integers(1024, 8193, size=batch))
    run_decode(device, 30 + batch, 32, 8, 128, lens)


@pytest.mark.parametrize("n_head,n_head_kv,lens", [(32, 8, [8192, 7000, 6000, 7800]), (28, 4, [4096] * 8),
                                                    (32, 8, [5000, 4500, 4100, 6000, 5900])])
def test_uniform_batches_8_splits(device, n_head, n_head_kv, lens):
    # batches of about one length (within 1.5x) of at least 4096 keys: at most 8 splits per sequence, each walking
    # several 32-key blocks per wave; every sequence and head checked
    run_decode(device, 50 + len(lens), n_head, n_head_kv, 128, lens)


def test_batch_over_launch_limit(device):
    # 40 sequences > 32 per launch: two launches reuse the workspace
    lens = list(np.random.default_rng(7).integers(1, 700, size=40))
    run_decode(device, 41, 8, 2, 64, lens, check_seqs=[0, 31, 32, 39])


# cfg4: Whisper large-v3-turbo: MHA self-attention over 1..448 positions, cross-attention over 1500 frames
@pytest.mark.parametrize("L", [1, 64, 224, 448])
def test_whisper_self(device, L):
    run_decode(device, 4 + L, 20, 20, 64, [L])


def test_whisper_self_beam5(device):
    run_decode(device, 45, 20, 20, 64, [448, 300, 17, 1, 129])


def test_whisper_cross_greedy(device):
    run_decode(device, 46, 20, 20, 64, [1500])


def test_whisper_cross_beam5_shared(device):
    # 5 beams as 5 query rows over ONE shared encoder cache (n_q = 5, non-causal)
    run_decode(device, 47, 20, 20, 64, [1500], n_q=5)


def test_whisper_cross_beam5_as_batch(device):
    # the same through 5 sequences that point at one cache
    run_decode(device, 48, 20, 20, 64, [1500] * 5, shared_cache=True)


@pytest.mark.parametrize("n_q,L", [(2, 2), (8, 8), (8, 300), (8, 1500)])
def test_causal_prompt_rows(device, n_q, L):
    # Whisper prompt rows (up to 8 per pass) appended at the end of the cache, each with its causal limit
    run_decode(device, 50 + n_q + L, 20, 20, 64, [L], n_q=n_q, causal=True)


@pytest.mark.parametrize("lens", [[700, 5], [8192, 5]])
@pytest.mark.parametrize("n_head,n_head_kv,hd", [(4, 1, 64), (7, 1, 128), (16, 1, 128), (32, 1, 64), (8, 8, 128)])
def test_group_sizes(device, n_head, n_head_kv, hd, lens):
    # 1..32 query heads per kv head: row tiles of 4, 8 and 16 rows, and several tiles; 8192 keys make 32 splits of 256
    # keys on 8-wave workgroups (at head dim 128 the merge that stripes the splits over the threads), 700 keys 6 (the
    # per-pair merge)
    run_decode(device, 60 + n_head + lens[0], n_head, n_head_kv, hd, lens)


def test_causal_gqa_multi_rowtile(device):
    run_decode(device, 70, 14, 2, 64, [900], n_q=6, causal=True)  # 42 rows per kv head: 3 tiles of 16


def test_padded_cache_stride(device):
    # caches with extra columns (a fused k|v row, say): kv_stride > n_head_kv * head_dim
    run_decode(device, 71, 8, 2, 128, [333, 1200], kv_pad=64)


@pytest.mark.parametrize("scale", [0.0, 0.3, 3.0])
def test_scale_semantics(device, scale):
    # scale 0 is uniform attention: the output is the mean of V (test_backend_ggml.cpp:715-735)
    out, _ = run_decode(device, 72, 4, 2, 64, [257], scale=scale)


def test_scale_zero_is_mean_of_v(device):
    rng = np.random.default_rng(73)
    L, hd = 1000, 64
    q = torch.from_numpy(normal_f16(rng, (1, 2 * hd))).to(device)
    k = torch.from_numpy(normal_f16(rng, (L, hd))).to(device)
    vn = normal_f16(rng, (L, hd))
    v = torch.from_numpy(vn).to(device)
    out, _ = A.decode(q, [k], [v], [L], n_head=2, n_head_kv=1, head_dim=hd, scale=0.0)
    mean = vn.astype(np.float64).mean(axis=0)
    got = out.cpu().numpy().astype(np.float64)
    np.testing.assert_allclose(got[0, :hd], mean, atol=2e-3)
    np.testing.assert_allclose(got[0, hd:], mean, atol=2e-3)


def test_split_count_invariance(device):
    # the merge must not depend on how the keys are split (test_whisper.cpp:255-270 checks cross_splits 1, 7, 64)
    rng = np.random.default_rng(74)
    L, hd = 4000, 128
    q = torch.from_numpy(normal_f16(rng, (1, 32 * hd))).to(device)
    k = torch.from_numpy(normal_f16(rng, (L, 8 * hd))).to(device)
    v = torch.from_numpy(normal_f16(rng, (L, 8 * hd))).to(device)
    outs = []
    plans = [dict(decode_max_workgroups=w) for w in (1, 7, 64, 100000)] + [dict(decode_splits=s) for s in (1, 7, 32)]
    for t in plans:
        o, l = A.decode(q, [k], [v], [L], n_head=32, n_head_kv=8, head_dim=hd, want_lse=True, tuning=t)
        outs.append((o.cpu().numpy().astype(np.float64), l.cpu().numpy()))
    for o, l in outs[1:]:
        assert np.abs(o - outs[0][0]).max() <= 2e-3
        assert np.abs(l - outs[0][1]).max() <= 1e-4


def test_decode_matches_prefill_kernel(device):
    # two independent kernels on one problem: the last query row of a causal prefill equals a decode step
    rng = np.random.default_rng(75)
    L, hd = 2500, 128
    qn = normal_f16(rng, (L, 28 * hd))
    k = torch.from_numpy(normal_f16(rng, (L, 4 * hd))).to(device)
    v = torch.from_numpy(normal_f16(rng, (L, 4 * hd))).to(device)
    q = torch.from_numpy(qn).to(device)
    po, pl = A.prefill(q, k, v, n_head=28, n_head_kv=4, head_dim=hd, want_lse=True)
    do, dl = A.decode(q[L - 1:L], [k], [v], [L], n_head=28, n_head_kv=4, head_dim=hd, want_lse=True)
    a = po[L - 1].cpu().numpy().astype(np.float64)
    b = do[0].cpu().numpy().astype(np.float64)
    assert np.abs(a - b).max() <= 2e-3
    assert np.abs(pl[L - 1].cpu().numpy() - dl[0].cpu().numpy()).max() <= 1e-3


# ---- mx_attn_decode_f32: the reference's f32 query rows and f32 output (query rounded to half in the kernel) ----

def run_decode_f32(device, seed, n_head, n_head_kv, hd, kv_lens, n_q=1, causal=False, shared_cache=False,
                   check_heads=None):
    rng = np.random.default_rng(seed)
    batch = len(kv_lens)
    kvw = n_head_kv * hd
    q = rng.standard_normal((batch * n_q, n_head * hd), dtype=np.float32)
    caches = []
    for b in range(batch):
        if shared_cache and b > 0:
            caches.append(caches[0])
            continue
        caches.append((normal_f16(rng, (kv_lens[b], kvw)), normal_f16(rng, (kv_lens[b], kvw))))
    scale = 1.0 / np.sqrt(hd)
    out, lse = A.decode(torch.from_numpy(q).to(device), [torch.from_numpy(k).to(device) for k, _ in caches],
                        [torch.from_numpy(v).to(device) for _, v in caches], list(kv_lens), n_head=n_head,
                        n_head_kv=n_head_kv, head_dim=hd, n_q=n_q, causal=causal, want_lse=True)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    out = out.cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy()
    qh = q.astype(np.float16)
    heads = np.arange(n_head) if check_heads is None else np.asarray(check_heads)
    cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
    for b in range(batch):
        k, v = caches[b]
        L = kv_lens[b]
        ro, rl = ref_attention(qh[b * n_q:(b + 1) * n_q], k, v, n_head, n_head_kv, hd, scale, p0=L - n_q,
                               causal=causal, heads=check_heads)
        assert_close(out[b * n_q:(b + 1) * n_q][:, cols], ro, hd, f"f32 seq {b} L={L}",
                     lse[b * n_q:(b + 1) * n_q][:, heads], rl)


def test_f32_whisper_cross_beam5(device):
    run_decode_f32(device, 41, 20, 20, 64, [1500], n_q=5)


def test_f32_whisper_prompt_rows(device):
    run_decode_f32(device, 42, 20, 20, 64, [9], n_q=4, causal=True)


def test_f32_llama3_8b_batch3(device):
    run_decode_f32(device, 43, 32, 8, 128, [1, 700, 5000], check_heads=[0, 13, 31])


@pytest.mark.parametrize("n_head,n_head_kv,hd,n_q", [(14, 2, 64, 1), (20, 20, 64, 5), (32, 8, 128, 4)])
def test_f32_many_splits(device, n_head, n_head_kv, hd, n_q):
    # 32 splits per tile on the f32 entry point (row tiles of 4, 8 and 16 rows; at head dim 128 the striped merge)
    run_decode_f32(device, 44 + n_q, n_head, n_head_kv, hd, [8192], n_q=n_q)


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("case", ["qwen513", "llama_b4", "whisper_cross_b5", "causal_rows", "gqa16_hd128"])
def test_waves_per_workgroup(device, waves, case):
    # both workgroup shapes (4 or 8 waves; the library picks 8 when a launch fits the CUs in one round) on every tile
    # size: rows per tile 4 (GQA 4), 8 (GQA 7, beam 5), 16 (causal rows, GQA 16)
    with A.tuning(decode_waves=waves):
        if case == "qwen513":
            run_decode(device, 1, 14, 2, 64, [513])
        elif case == "llama_b4":
            run_decode(device, 34, 32, 8, 128, [6841, 1638, 33, 2721], check_heads=[0, 5, 31])
        elif case == "whisper_cross_b5":
            run_decode(device, 95, 20, 20, 64, [1500] * 5, n_q=1, shared_cache=True, check_heads=[0, 7, 19])
        elif case == "causal_rows":
            run_decode(device, 108, 14, 2, 64, [300], n_q=8, causal=True)
        else:
            run_decode(device, 114, 16, 1, 128, [777])


def test_workspace_shared_across_shapes(device):
    """One workspace (sized for the largest call) serving calls of different shapes in turn, as a decoder's workspace
    serves decode steps, batches and prompt chunks: a call's partials must never land where another call's split
    counters lie. Every call is compared bit for bit with the same call on a fresh workspace."""
    rng = np.random.default_rng(2024)
    calls = [(32, 8, 128, [8192], 1, False), (32, 8, 128, [6841, 1638, 4000, 2721], 1, False),
             (28, 4, 128, [3000], 64, True), (32, 8, 128, [700], 1, False), (14, 2, 64, [2000, 513], 1, False),
             (32, 8, 128, [5000] * 6, 1, False), (28, 4, 128, [3000], 64, True)]
    need = max(A.decode_workspace_bytes(n_head=nh, n_head_kv=nkv, head_dim=hd, n_q=nq, batch=len(lens),
                                        max_kv_len=max(lens), causal=c) for nh, nkv, hd, lens, nq, c in calls)
    shared = A.new_workspace(need, device)
    for nh, nkv, hd, lens, nq, c in calls:
        q = torch.from_numpy(normal_f16(rng, (len(lens) * nq, nh * hd))).to(device)
        k = [torch.from_numpy(normal_f16(rng, (L, nkv * hd))).to(device) for L in lens]
        v = [torch.from_numpy(normal_f16(rng, (L, nkv * hd))).to(device) for L in lens]
        kw = dict(n_head=nh, n_head_kv=nkv, head_dim=hd, n_q=nq, causal=c, want_lse=True)
        got, gl = A.decode(q, k, v, lens, workspace=shared, **kw)
        ref, rl = A.decode(q, k, v, lens, **kw)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"{nh}/{nkv} {lens} n_q {nq}"
        assert torch.equal(gl.view(torch.int32), rl.view(torch.int32))
