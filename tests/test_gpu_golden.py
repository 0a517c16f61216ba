"""GPU parity on the committed fixtures: the CPU plumbing case (Qwen2.5-7B
attention shape, 256 local causal + 256 peer, fp16 inputs) through the HIP
kernels -- ring_attn_with_lse for both segments and merge_attn_states with
prefix = peer, suffix = local (ring_backend.py:354) -- against the float64
fixture, at the fp16 gates (out 2e-3, LSE 1e-3)."""

import math

import pytest
import torch

from hcp_vllm_plugin_amd import merge_attn_states, ring_attn_with_lse
from tests._util import max_err
from tests.golden_util import plumbing_inputs

pytestmark = pytest.mark.gpu


def test_plumbing_fixture_on_hip(dev):
    (q, kl, vl, kp, vp), fx = plumbing_inputs()
    q, kl, vl, kp, vp = (t.to(dev) for t in (q, kl, vl, kp, vp))
    scale = 1.0 / math.sqrt(128)
    sub = int(fx["sub"])
    o_l, l_l = ring_attn_with_lse(q, kl, vl, scale, 0)
    o_p, l_p = ring_attn_with_lse(q, kp, vp, scale, None)
    out = torch.empty_like(o_l)
    merge_attn_states(out, o_p, l_p, o_l, l_l)
    torch.cuda.synchronize()
    assert max_err(l_l, torch.from_numpy(fx["lse_local"])) <= 1e-3
    assert max_err(l_p, torch.from_numpy(fx["lse_peer"])) <= 1e-3
    assert max_err(o_l[::sub], torch.from_numpy(fx["out_local"])) <= 2e-3
    assert max_err(o_p[::sub], torch.from_numpy(fx["out_peer"])) <= 2e-3
    assert max_err(out[::sub], torch.from_numpy(fx["out_merged"])) <= 2e-3
