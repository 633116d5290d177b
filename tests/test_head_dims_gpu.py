"""Every head dim the reference's llama decoder accepts (powers of two in [4, 256], metal_llama_decoder.mm:432-435),
through every attention entry point of the C ABI, against the f64 oracle.

Head dims 64 and 128 run on the matrix-core kernels and are covered by the other test files; 256 runs on them too (its
own instantiations: 4-wave decode and prefill workgroups), and 4 .. 32 on the per-query kernel (small.hip). The
reference's own default tiny model (tests/unit/test_metal_llama_decoder.cpp:56-57: 4 q / 2 kv heads, head_dim 16) is
driven the way that test drives its decoder (:497-532): a 45-token prompt in chunks of 20 on the reference's f32
q|k|v rows, then decode steps, each against the oracle over the cache as written. Tolerance as everywhere (helpers).
"""
import numpy as np
import pytest
import torch

from dooms_amd import _lib
from dooms_amd import attention as A
from helpers import assert_close, ref_attention
from oracle import oracle as O
from test_decode_gpu import run_decode, run_decode_f32
from test_decode_rope_gpu import run_rope
from test_prefill_gpu import check_prefill
from test_prefill_rope_gpu import run_prefill_rope

pytestmark = pytest.mark.gpu

SMALL = [4, 8, 16, 32]


@pytest.mark.parametrize("hd", SMALL + [256])
@pytest.mark.parametrize("lens", [[1], [45], [700], [3000, 17, 129]])
def test_decode_head_dims(device, hd, lens):
    run_decode(device, hd + sum(lens), 4, 2, hd, lens)


@pytest.mark.parametrize("hd", SMALL + [256])
def test_decode_causal_rows_and_f32(device, hd):
    run_decode(device, 3 + hd, 8, 2, hd, [300, 64], n_q=6, causal=True)
    run_decode_f32(device, 4 + hd, 8, 8, hd, [1500, 1500], n_q=3)


@pytest.mark.parametrize("hd", SMALL + [256])
@pytest.mark.parametrize("N,chunk", [(45, None), (45, 20), (300, 128), (1000, None)])
def test_prefill_head_dims(device, hd, N, chunk):
    check_prefill(device, hd + N, N, 4, 2, hd, chunk=chunk)


@pytest.mark.parametrize("hd", SMALL + [256])
def test_prefill_noncausal_and_negative_scale(device, hd):
    check_prefill(device, 7 + hd, 200, 6, 3, hd, causal=False)
    check_prefill(device, 8 + hd, 150, 4, 4, hd, scale=-0.2)


@pytest.mark.parametrize("hd", SMALL + [256])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_rope_entry_points(device, hd, mode):
    run_prefill_rope(device, 20 + hd + mode, 4, 2, hd, 37, 11, mode, 10000.0)
    run_rope(device, 30 + hd + mode, 4, 2, hd, [1, 70, 600], mode, 10000.0)


@pytest.mark.parametrize("hd", SMALL + [256])
def test_workspace_entry_points(device, hd):
    # mx_attn_prefill_ws / _rope_ws and mx_attn_decode_noalloc at every head dim (the small ones need no workspace)
    check_prefill(device, 40 + hd, 64, 8, 2, hd, chunk=16, workspace="auto")
    run_prefill_rope(device, 41 + hd, 8, 2, hd, 16, 100, 0, 500000.0, workspace="auto")


def test_reference_tiny_model_prompt_then_steps(device):
    """The reference's default tiny llama shape (4 q / 2 kv heads, head_dim 16, test_metal_llama_decoder.cpp:56-57)
    fed as its decoder test feeds it (:497-532): a 45-token prompt in chunks of 20 on f32 q|k|v rows (mx_attn_prefill_rope
    writes the rotated keys/values), then 8 decode steps (mx_attn_decode_rope appends each), for both rotary layouts.
    Every call's output is checked against the oracle over the cache as the calls left it."""
    for mode, base in ((0, 10000.0), (1, 1000000.0)):
        rng = np.random.default_rng(500 + mode)
        nh, nkv, hd, n_ctx = 4, 2, 16, 64
        qw, kvw = nh * hd, nkv * hd
        dk = torch.zeros(n_ctx, kvw, dtype=torch.float16, device=device)
        dv = torch.zeros(n_ctx, kvw, dtype=torch.float16, device=device)
        rows = rng.standard_normal((53, qw + 2 * kvw), dtype=np.float32)
        scale = 1.0 / np.sqrt(hd)

        def check(out, lse, t0, n):
            gk, gv = dk.cpu().numpy(), dv.cpu().numpy()
            q = np.stack([O.rope_f32(rows[t0 + i, :qw], mode, base, hd, t0 + i) for i in range(n)]).astype(np.float16)
            ro, rl = ref_attention(q, gk[:t0 + n], gv[:t0 + n], nh, nkv, hd, scale, p0=t0, causal=True)
            assert_close(out.cpu().numpy().astype(np.float64), ro, hd, f"rows {t0}..{t0 + n - 1}",
                         lse.cpu().numpy(), rl)

        for p0 in range(0, 45, 20):
            m = min(20, 45 - p0)
            out, lse = A.prefill_rope(torch.from_numpy(rows[p0:p0 + m]).to(device), dk, dv, n_head=nh, n_head_kv=nkv,
                                      head_dim=hd, rope_mode=mode, rope_base=base, p0=p0, n_kv=n_ctx,
                                      want_lse=True)
            torch.cuda.synchronize()
            check(out, lse, p0, m)
        for p in range(45, 53):
            out, lse = A.decode_rope(torch.from_numpy(rows[p:p + 1]).to(device), [dk], [dv], [p + 1], n_head=nh,
                                     n_head_kv=nkv, head_dim=hd, rope_mode=mode, rope_base=base, want_lse=True)
            torch.cuda.synchronize()
            check(out, lse, p, 1)


def test_gemma2_9b_shape_hd256(device):
    # head_dim 256 at a real model's shape (16 q / 8 kv heads): a decode over 8192 keys and a 1024-token prompt
    run_decode(device, 256, 16, 8, 256, [8192], check_heads=[0, 1, 7, 15])
    check_prefill(device, 257, 1024, 16, 8, 256, rows=list(range(0, 1024, 37)) + [1023], heads=[0, 3, 8, 15])


@pytest.mark.parametrize("hd", [2, 12, 48, 80, 512])
def test_other_head_dims_refused(device, hd):
    q = torch.zeros(4, 4 * hd + 8, dtype=torch.float16, device=device)
    with pytest.raises(_lib.MxAttnError) as e:
        A.prefill(q, q, q, n_head=4, n_head_kv=4, head_dim=hd)
    assert e.value.code in (_lib.UNSUPPORTED, _lib.INVALID_ARGUMENT)
