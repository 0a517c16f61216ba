"""The oracle against the committed golden fixtures (tests/golden/), which
make_golden.py computed by a separate route (vectorised float64 numpy)."""

import math

import numpy as np
import torch

from oracle import ring_oracle as orc
from tests.golden_util import load, plumbing_inputs


def test_oracle_matches_micro_fixture():
    fx = load("micro.npz")
    q, k, v = (torch.from_numpy(fx[n]).float() for n in ("q", "k", "v"))
    for name, off in (("c0", 0), ("c3", 3), ("nc", None)):
        o, lse = orc.attn_with_lse(q, k, v, float(fx["scale"]), off)
        np.testing.assert_allclose(o.numpy(), fx[f"out_{name}"], atol=2e-6)
        np.testing.assert_allclose(lse.numpy(), fx[f"lse_{name}"], atol=2e-6)


def test_oracle_matches_plumbing_fixture():
    (q, kl, vl, kp, vp), fx = plumbing_inputs()
    scale = 1.0 / math.sqrt(128)
    sub = int(fx["sub"])
    o_l, l_l = orc.attn_with_lse(q.float(), kl.float(), vl.float(), scale, 0)
    o_p, l_p = orc.attn_with_lse(q.float(), kp.float(), vp.float(), scale, None)
    o_m = orc.lse_merge(o_l, l_l, o_p, l_p)
    np.testing.assert_allclose(l_l.numpy(), fx["lse_local"], atol=2e-5)
    np.testing.assert_allclose(l_p.numpy(), fx["lse_peer"], atol=2e-5)
    np.testing.assert_allclose(o_l[::sub].numpy(), fx["out_local"], atol=2e-5)
    np.testing.assert_allclose(o_p[::sub].numpy(), fx["out_peer"], atol=2e-5)
    np.testing.assert_allclose(o_m[::sub].numpy(), fx["out_merged"], atol=2e-5)
    # merge_pair's merged LSE is the LSE of the union of keys
    _, l_m = orc.merge_pair(o_l, l_l, o_p, l_p)
    full = torch.logaddexp(torch.from_numpy(fx["lse_local"]), torch.from_numpy(fx["lse_peer"]))
    np.testing.assert_allclose(l_m.numpy(), full.numpy(), atol=2e-5)
