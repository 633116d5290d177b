"""The committed golden fixtures (tests/golden/*.npz) through both HIP entry points, against the fixture outputs."""
import glob
import os

import numpy as np
import pytest
import torch

from dooms_amd import attention as A
from helpers import assert_close

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))


@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
def test_fixture_prefill(device, path):
    z = np.load(path)
    n_head, n_head_kv, hd, n_q, n_kv, p0, causal = (int(x) for x in z["meta"])
    q, k, v = (torch.from_numpy(z[n]).to(device) for n in ("q", "k", "v"))
    out, lse = A.prefill(q, k, v, n_head=n_head, n_head_kv=n_head_kv, head_dim=hd, p0=p0, n_kv=n_kv,
                         causal=bool(causal), scale=float(z["scale"]), want_lse=True)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), z["out"], hd, os.path.basename(path), lse.cpu().numpy(), z["lse"])


@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
def test_fixture_decode(device, path):
    z = np.load(path)
    n_head, n_head_kv, hd, n_q, n_kv, p0, causal = (int(x) for x in z["meta"])
    if causal and p0 != n_kv - n_q:
        pytest.skip("decode rows sit at the end of the cache")
    q, k, v = (torch.from_numpy(z[n]).to(device) for n in ("q", "k", "v"))
    out, lse = A.decode(q, [k], [v], [n_kv], n_head=n_head, n_head_kv=n_head_kv, head_dim=hd, n_q=n_q,
                        causal=bool(causal), scale=float(z["scale"]), want_lse=True)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), z["out"], hd, os.path.basename(path), lse.cpu().numpy(), z["lse"])
