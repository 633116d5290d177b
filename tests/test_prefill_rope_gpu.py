"""Parity of mx_attn_prefill_rope (the reference's prompt path: rope_store of the chunk's keys/values, then flash
attention of f32 query rows rotated in the kernel, f32 output) with the oracle, through the C ABI.

Replaces rope_store + attention_prefill (llama_kernels.h:520-545, 632-769; metal_llama_decoder.mm:276-296). Checked: the
written key rows against oracle_rope_f32 rounded to half (within one half ulp, or an f32
rotation's error near zero), the value rows bit for bit, every other
cache row untouched, and the output against the f64 attention oracle over the cache as the kernel left it, with the
query rotated by the oracle and rounded to half (as the reference rounds q at llama_kernels.h:660).
"""
import numpy as np
import pytest
import torch

from dooms_amd import attention as A
from helpers import assert_close, ref_attention
from oracle import oracle as O
from test_decode_rope_gpu import assert_key_rotated

pytestmark = pytest.mark.gpu


def run_prefill_rope(device, seed, n_head, n_head_kv, hd, M, p0, mode, base, spare=5, rows=None, heads=None,
                     qkv_pad=0, kv_pad=0, n_kv=None, causal=True, workspace=None):
    rng = np.random.default_rng(seed)
    qw, kvw = n_head * hd, n_head_kv * hd
    qkv = rng.standard_normal((M, qw + 2 * kvw + qkv_pad), dtype=np.float32)
    cap = p0 + M + spare
    kc = rng.standard_normal((cap, kvw + kv_pad), dtype=np.float32).astype(np.float16)
    vc = rng.standard_normal((cap, kvw + kv_pad), dtype=np.float32).astype(np.float16)
    dk, dv = torch.from_numpy(kc).to(device), torch.from_numpy(vc).to(device)
    scale = 1.0 / np.sqrt(hd)
    out, lse = A.prefill_rope(torch.from_numpy(qkv).to(device), dk, dv, n_head=n_head, n_head_kv=n_head_kv,
                              head_dim=hd, rope_mode=mode, rope_base=base, p0=p0, n_kv=n_kv, causal=causal,
                              want_lse=True, workspace=workspace)
    torch.cuda.synchronize()
    out = out.cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy()
    gk, gv = dk.cpu().numpy(), dv.cpu().numpy()
    q_rot = np.empty((M, qw), dtype=np.float16)
    for t in range(M):
        pos = p0 + t
        q_rot[t] = O.rope_f32(qkv[t, :qw], mode, base, hd, pos).astype(np.float16)
        k_rot = O.rope_f32(qkv[t, qw:qw + kvw], mode, base, hd, pos)
        assert_key_rotated(gk[pos, :kvw], qkv[t, qw:qw + kvw], k_rot, mode, hd, f"row {t}")
        assert np.array_equal(gv[pos, :kvw].view(np.int16),
                              qkv[t, qw + kvw:qw + 2 * kvw].astype(np.float16).view(np.int16)), f"row {t}: value"
    others = np.ones(cap, dtype=bool)
    others[p0:p0 + M] = False
    assert np.array_equal(gk[others].view(np.int16), kc[others].view(np.int16)), "key rows outside the chunk touched"
    assert np.array_equal(gv[others].view(np.int16), vc[others].view(np.int16)), "value rows outside the chunk touched"
    assert np.array_equal(gk[:, kvw:].view(np.int16), kc[:, kvw:].view(np.int16)), "key row padding touched"
    nk = (p0 + M) if n_kv is None else n_kv
    ro, rl = ref_attention(q_rot, gk[:nk, :kvw], gv[:nk, :kvw], n_head, n_head_kv, hd, scale, p0=p0, causal=causal,
                           rows=rows, heads=heads)
    r = np.arange(M) if rows is None else np.asarray(rows)
    h = np.arange(n_head) if heads is None else np.asarray(heads)
    cols = np.concatenate([np.arange(x * hd, (x + 1) * hd) for x in h])
    assert_close(out[r][:, cols], ro, hd, f"M={M} p0={p0}", lse[r][:, h], rl)


# cfg2: Qwen2.5-0.5B 512-token prompt (neox, base 1e6)
def test_qwen05b_prompt_512(device):
    run_prefill_rope(device, 1, 14, 2, 64, 512, 0, 1, 1000000.0, rows=list(range(0, 512, 7)) + [511])


# Llama-3-8B chunk after 100 cached positions
def test_llama3_8b_chunk_at_100(device):
    run_prefill_rope(device, 2, 32, 8, 128, 300, 100, 0, 500000.0, rows=[0, 1, 63, 64, 150, 255, 256, 299],
                     heads=[0, 3, 4, 31])


# a chunk deep into a 32k context: large rotation angles
def test_qwen7b_chunk_at_30000(device):
    run_prefill_rope(device, 3, 28, 4, 128, 96, 30000, 1, 1000000.0, rows=[0, 31, 32, 95], heads=[0, 7, 27])


# Whisper prompt: no rotation, MHA
def test_whisper_prompt_no_rope(device):
    run_prefill_rope(device, 4, 20, 20, 64, 5, 0, 2, 0.0)


@pytest.mark.parametrize("M,p0", [(1, 0), (1, 37), (33, 0), (65, 3)])
def test_small_chunks(device, M, p0):
    run_prefill_rope(device, 10 + M + p0, 8, 2, 64, M, p0, 0, 10000.0)


def test_padded_strides(device):
    run_prefill_rope(device, 5, 8, 2, 128, 40, 9, 1, 10000.0, qkv_pad=16, kv_pad=8)


def test_prompt_in_chunks_matches_one_call(device):
    # the reference's chunked prompt (test_metal_llama_decoder.cpp:497-532: 45 tokens in chunks of 20)
    rng = np.random.default_rng(6)
    nh, nkv, hd, N = 4, 2, 64, 45
    qkv = torch.from_numpy(rng.standard_normal((N, (nh + 2 * nkv) * hd), dtype=np.float32)).to(device)
    caches = [(torch.zeros(N, nkv * hd, dtype=torch.float16, device=device),
               torch.zeros(N, nkv * hd, dtype=torch.float16, device=device)) for _ in range(2)]
    one, _ = A.prefill_rope(qkv, *caches[0], n_head=nh, n_head_kv=nkv, head_dim=hd, rope_mode=0)
    parts = []
    for p0 in range(0, N, 20):
        o, _ = A.prefill_rope(qkv[p0:p0 + 20], *caches[1], n_head=nh, n_head_kv=nkv, head_dim=hd, rope_mode=0,
                              p0=p0, n_kv=min(N, p0 + 20))
        parts.append(o)
    torch.cuda.synchronize()
    assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])
    # per row the same keys in the same block order: the chunked result equals the one-call result
    assert torch.equal(torch.cat(parts), one)


# the reference's prompt path under every workgroup plan (see test_prefill_gpu.test_workgroup_plans)
@pytest.mark.parametrize("plan", [2, 4, 8])
def test_workgroup_plans(device, plan):
    with A.tuning(prefill_plan=plan):
        run_prefill_rope(device, 300, 14, 2, 64, 300, 170, 1, 1000000.0)
        run_prefill_rope(device, 301, 8, 2, 128, 200, 0, 0, 500000.0)


# mx_attn_prefill_rope_ws: chunks of few rows take the split-KV kernel (keys/values cached and queries rotated by
# rope_store, then the decode kernel on the f32 query rows); larger ones the flash kernel
@pytest.mark.parametrize("n_head,n_head_kv,hd,M,p0,mode", [(32, 8, 128, 1, 4000, 0), (32, 8, 128, 16, 4000, 0),
                                                           (28, 4, 128, 64, 3000, 1), (14, 2, 64, 200, 100, 1),
                                                           (8, 8, 64, 40, 0, 2)])
def test_prefill_rope_ws(device, n_head, n_head_kv, hd, M, p0, mode):
    heads = [0, n_head // 2, n_head - 1]
    run_prefill_rope(device, 600 + M, n_head, n_head_kv, hd, M, p0, mode, 500000.0, heads=heads, workspace="auto")
