"""The prefill kernel's softmax bookkeeping under score patterns that move the row maximum: the kernel keeps a
reference maximum and takes the exact update only when a block's probabilities at that reference sum above 2^8 (or
overflow), so these inputs drive that path in every block (scores rising along the keys), never after the first
(falling), or at isolated keys (spikes), for every plan and head dim. Checked against the f64 oracle with the usual
tolerance (helpers.assert_close, LSE included). Mirrors the reference's own softmax with the running maximum
(attention_prefill, llama_kernels.h:632-769), whose results do not depend on where the maximum sits."""
import numpy as np
import pytest
import torch

from dooms_amd import attention as A
from helpers import assert_close, ref_attention

pytestmark = pytest.mark.gpu


def patterned(rng, N, n_head, n_head_kv, hd, kind):
    """q rows along a common direction u, keys t_j u + noise: the scaled scores follow t_j (about 33 t_j in base-2
    units at head dim 128)."""
    u = np.ones(hd, np.float32)
    j = np.arange(N, dtype=np.float32)
    if kind == "rising":
        t = 3.0 * j / N
    elif kind == "falling":
        t = 3.0 * (1.0 - j / N)
    else:  # spikes: every 37th key well above its neighbours, growing along the prompt
        t = np.where(j % 37 == 5, 1.0 + 2.0 * j / N, 0.0)
    q = np.tile(2.0 * u, (N, n_head)) + rng.standard_normal((N, n_head * hd)).astype(np.float32) * 0.3
    k = (t[:, None, None] * u[None, None, :] +
         rng.standard_normal((N, n_head_kv, hd)).astype(np.float32) * 0.3).reshape(N, n_head_kv * hd)
    v = rng.standard_normal((N, n_head_kv * hd)).astype(np.float32)
    return [a.astype(np.float16) for a in (q, k, v)]


@pytest.mark.parametrize("kind", ["rising", "falling", "spikes"])
@pytest.mark.parametrize("hd,n_head,n_head_kv,plan", [(128, 8, 2, 8), (128, 8, 2, 4), (128, 8, 2, 2), (64, 14, 2, 8),
                                                      (64, 14, 2, 2), (256, 4, 2, 0)])
def test_prefill_score_patterns(device, kind, hd, n_head, n_head_kv, plan):
    rng = np.random.default_rng(hd + n_head + plan)
    N = 640
    q, k, v = patterned(rng, N, n_head, n_head_kv, hd, kind)
    dq, dk, dv = [torch.from_numpy(a).to(device) for a in (q, k, v)]
    scale = 1.0 / np.sqrt(hd)
    out, lse = A.prefill(dq, dk, dv, n_head=n_head, n_head_kv=n_head_kv, head_dim=hd, scale=scale, want_lse=True,
                         tuning={"prefill_plan": plan} if plan else None)
    torch.cuda.synchronize()
    rows = np.r_[0:8, 60:70, 250:260, N - 16:N]
    ro, rl = ref_attention(q, k, v, n_head, n_head_kv, hd, scale, causal=True, rows=rows)
    assert_close(out.cpu().numpy()[rows], ro, hd, f"{kind} hd {hd} plan {plan}", lse.cpu().numpy()[rows], rl)


@pytest.mark.parametrize("kind", ["rising", "spikes"])
def test_prefill_score_patterns_chunked_stream(device, kind):
    """The same patterns in chunks against the growing cache, through the workspace entry point (the stream-K split
    forced where it applies), so that partial tiles merge references set in different launches."""
    rng = np.random.default_rng(7)
    N, n_head, n_head_kv, hd = 1024, 14, 2, 64
    q, k, v = patterned(rng, N, n_head, n_head_kv, hd, kind)
    dq, dk, dv = [torch.from_numpy(a).to(device) for a in (q, k, v)]
    out = torch.empty(N, n_head * hd, dtype=torch.float16, device=device)
    lse = torch.empty(N, n_head, dtype=torch.float32, device=device)
    for p0 in range(0, N, 256):
        A.prefill(dq[p0:p0 + 256], dk[:p0 + 256], dv[:p0 + 256], n_head=n_head, n_head_kv=n_head_kv, head_dim=hd,
                  p0=p0, out=out[p0:p0 + 256], lse=lse[p0:p0 + 256], workspace="auto",
                  tuning={"prefill_stream": 1})
    torch.cuda.synchronize()
    rows = np.r_[0:4, 300:310, 700:710, N - 8:N]
    ro, rl = ref_attention(q, k, v, n_head, n_head_kv, hd, 1.0 / np.sqrt(hd), causal=True, rows=rows)
    assert_close(out.cpu().numpy()[rows], ro, hd, f"{kind} chunked", lse.cpu().numpy()[rows], rl)
