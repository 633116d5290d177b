"""Parity of mx_attn_decode_rope (the fused decode step: rotary embedding of the new token's q and k, its k/v appended
to the caches, decode attention) with the oracle, through the C ABI.

Replaces the reference's `attention` kernel with fused_rope = 1 (llama_kernels.h:552-630) and rope_store followed by
split attention (llama_kernels.h:521-549, 856-929). Checked: the output against the f64 attention oracle over the cache
with the new row in place (the query rotated by oracle_rope_f32 and rounded to half, as the kernel hands it to the
matrix cores), the written key row against the oracle's rotated key rounded to half (within one half ulp: the angle's
sine and cosine may round differently; near zero, within an f32 rotation's error, assert_key_rotated), the value row bit for bit, and every other cache row untouched.
Shapes: Llama-3-8B (normal rope, base 500000), Qwen2.5-0.5B (neox, base 1e6), Whisper self-attention (no rope).
"""
import numpy as np
import pytest
import torch

from dooms_amd import _lib
from dooms_amd import attention as A
from helpers import assert_close, ref_attention
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def half_ulps(a, b):
    """Distance in units of the last place between two f16 arrays of finite values."""
    ia = a.view(np.int16).astype(np.int32)
    ib = b.view(np.int16).astype(np.int32)
    ia = np.where(ia < 0, -32768 - ia, ia)  # sign-magnitude -> ordered integers
    ib = np.where(ib < 0, -32768 - ib, ib)
    return np.abs(ia - ib)


def assert_key_rotated(got, x, rot, mode, hd, msg):
    """The written key row (f16) against the oracle's rotation rot (f32) of the unrotated row x (f32): within one half
    ulp of rot rounded to half, or, where the rotated value is small beside its pair's operands (a x0 cos - x1 sin that
    nearly cancels), within an f32-level absolute error of those operands. The reference rotates in f32
    (llama_kernels.h:508-518), so an f32 rotation is that far from the exact one; a wrong angle, pair or sign is
    orders of magnitude beyond both bounds."""
    ulps = half_ulps(got, rot.astype(np.float16))
    h = x.reshape(-1, hd)
    if mode == 0:
        partner = h.reshape(-1, hd // 2, 2)[:, :, ::-1].reshape(h.shape)
    elif mode == 1:
        partner = np.roll(h, hd // 2, axis=1)
    else:
        partner = np.zeros_like(h)
    mag = np.maximum(np.abs(h), np.abs(partner)).ravel().astype(np.float64)
    err = np.abs(got.astype(np.float64) - rot.astype(np.float64))
    bad = (ulps > 1) & (err > 2.0 ** -20 * mag)
    assert not bad.any(), (f"{msg}: key element {int(np.argmax(bad))} off by {int(ulps[bad].max())} half ulps, "
                           f"error {err[bad].max():.3g}")


def run_rope(device, seed, n_head, n_head_kv, hd, kv_lens, mode, base, spare=3, qkv_pad=0, kv_pad=0,
             check_heads=None, poison=False):
    rng = np.random.default_rng(seed)
    batch = len(kv_lens)
    qw, kvw = n_head * hd, n_head_kv * hd
    qkv = rng.standard_normal((batch, qw + 2 * kvw + qkv_pad), dtype=np.float32)
    kc = [rng.standard_normal((L + spare, kvw + kv_pad), dtype=np.float32).astype(np.float16) for L in kv_lens]
    vc = [rng.standard_normal((L + spare, kvw + kv_pad), dtype=np.float32).astype(np.float16) for L in kv_lens]
    if poison:
        # the row the step appends and the spare rows behind it hold Inf and NaN half patterns (fresh or pooled
        # memory): the kernel must not let any of them reach the output
        pats = np.array([0x7C00, 0xFC00, 0x7E00, 0xFFFF, 0x7C01], dtype=np.uint16)
        for b, L in enumerate(kv_lens):
            for c in (kc[b], vc[b]):
                tail = c[L - 1:].view(np.uint16)
                tail[...] = pats[np.arange(tail.size).reshape(tail.shape) % len(pats)]
    dk = [torch.from_numpy(k).to(device) for k in kc]
    dv = [torch.from_numpy(v).to(device) for v in vc]
    scale = 1.0 / np.sqrt(hd)
    out, lse = A.decode_rope(torch.from_numpy(qkv).to(device), dk, dv, list(kv_lens), n_head=n_head,
                             n_head_kv=n_head_kv, head_dim=hd, rope_mode=mode, rope_base=base, want_lse=True)
    torch.cuda.synchronize()
    out = out.cpu().numpy().astype(np.float64)
    lse = lse.cpu().numpy()
    for b, L in enumerate(kv_lens):
        pos = L - 1
        q_rot = O.rope_f32(qkv[b, :qw], mode, base, hd, pos).astype(np.float16)[None, :]
        k_rot = O.rope_f32(qkv[b, qw:qw + kvw], mode, base, hd, pos)
        v_new = qkv[b, qw + kvw:qw + 2 * kvw].astype(np.float16)
        gk, gv = dk[b].cpu().numpy(), dv[b].cpu().numpy()
        # the appended row, and nothing else written
        assert_key_rotated(gk[pos, :kvw], qkv[b, qw:qw + kvw], k_rot, mode, hd, f"seq {b}")
        assert np.array_equal(gv[pos, :kvw].view(np.int16), v_new.view(np.int16)), f"seq {b}: value row differs"
        others = np.ones(L + spare, dtype=bool)
        others[pos] = False
        assert np.array_equal(gk[others].view(np.int16), kc[b][others].view(np.int16)), f"seq {b}: key rows touched"
        assert np.array_equal(gv[others].view(np.int16), vc[b][others].view(np.int16)), f"seq {b}: value rows touched"
        assert np.array_equal(gk[pos, kvw:].view(np.int16), kc[b][pos, kvw:].view(np.int16))
        # attention over the cache as the kernel left it (the key row within an ulp of the oracle's)
        ro, rl = ref_attention(q_rot, gk[:L, :kvw], gv[:L, :kvw], n_head, n_head_kv, hd, scale, causal=False,
                               heads=check_heads)
        heads = np.arange(n_head) if check_heads is None else np.asarray(check_heads)
        cols = np.concatenate([np.arange(h * hd, (h + 1) * hd) for h in heads])
        assert_close(out[b:b + 1, cols], ro, hd, f"seq {b} L={L}", lse[b:b + 1, heads], rl)


# Llama-3-8B: the new position in every place of the split/wave/block walk
@pytest.mark.parametrize("L", [1, 2, 17, 32, 33, 128, 129, 300, 4097, 8192])
def test_llama3_8b_rope_decode(device, L):
    run_rope(device, L, 32, 8, 128, [L], 0, 500000.0, check_heads=[0, 5, 17, 31] if L > 4000 else None)


def test_llama3_8b_rope_decode_batch4(device):
    rng = np.random.default_rng(7)
    lens = [int(x) for x in rng.integers(1024, 8193, size=4)]
    run_rope(device, 8, 32, 8, 128, lens, 0, 500000.0, check_heads=[0, 9, 30])


def test_qwen05b_rope_decode_513(device):
    run_rope(device, 2, 14, 2, 64, [513], 1, 1000000.0)


def test_qwen7b_rope_decode_32k(device):
    # the fused step over 64 splits (4 kv heads at 32768 keys), the new row in the last split
    run_rope(device, 5, 28, 4, 128, [32768], 1, 1000000.0, check_heads=[0, 13, 27])


@pytest.mark.parametrize("L", [1, 64, 65, 1000])
def test_neox_hd128_rope_decode(device, L):
    run_rope(device, 30 + L, 28, 4, 128, [L], 1, 1000000.0)


def test_whisper_self_attention_step_no_rope(device):
    run_rope(device, 3, 20, 20, 64, [1, 7, 448, 200, 33], 2, 0.0)


def test_rope_decode_padded_strides(device):
    run_rope(device, 4, 8, 2, 64, [77, 300], 0, 10000.0, qkv_pad=16, kv_pad=8)


def test_rope_decode_rejects_shared_cache(device):
    k = torch.zeros(16, 128, dtype=torch.float16, device=device)
    v = torch.zeros(16, 128, dtype=torch.float16, device=device)
    qkv = torch.zeros(2, 4 * 64 + 2 * 128, dtype=torch.float32, device=device)
    with pytest.raises(_lib.MxAttnError) as e:
        A.decode_rope(qkv, [k, k], [v, v], [4, 5], n_head=4, n_head_kv=2, head_dim=64, rope_mode=0)
    assert e.value.code == _lib.INVALID_ARGUMENT


# the new position in every wave of both workgroup shapes (4 or 8 waves of 32-key blocks per split)
@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("L", [33, 100, 129, 200, 257, 8192])
def test_rope_decode_waves_per_workgroup(device, waves, L):
    with A.tuning(decode_waves=waves):
        run_rope(device, 500 + L, 32, 8, 128, [L], 0, 500000.0, check_heads=[0, 5, 17, 31] if L > 4000 else None)


# The appended row and the rows past it start as Inf / NaN: masked key slots of the last block are clamped to the new
# row, and nothing read from that row's memory (stale, and being overwritten) may reach the output.
@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("L", [1, 2, 33, 129, 8192])
def test_rope_decode_poisoned_tail(device, waves, L):
    with A.tuning(decode_waves=waves):
        run_rope(device, 900 + L, 32, 8, 128, [L], 0, 500000.0, spare=40, poison=True,
                 check_heads=[0, 5, 17, 31] if L > 4000 else None)


@pytest.mark.parametrize("L", [1, 2, 65, 513])
def test_rope_decode_poisoned_tail_hd64(device, L):
    run_rope(device, 950 + L, 14, 2, 64, [L], 1, 1000000.0, spare=40, poison=True)
