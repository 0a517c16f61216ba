"""Loads the committed golden fixtures (tests/golden/*.npz) and regenerates
their seeded inputs exactly as tests/golden/make_golden.py drew them."""

import hashlib
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(GOLDEN, name), allow_pickle=False))


def plumbing_inputs():
    """q [256,28,128], k_local, v_local, k_peer, v_peer [256,4,128], fp16 (CPU),
    checked against the fixture's input SHA-256."""
    h, hkv, d, n = 28, 4, 128, 256
    gen = torch.Generator().manual_seed(0)
    shapes = [(n, h, d), (n, hkv, d), (n, hkv, d), (n, hkv, d), (n, hkv, d)]
    ts = [torch.randn(*s, generator=gen).to(torch.float16) for s in shapes]
    sha = hashlib.sha256(b"".join(t.numpy().tobytes() for t in ts)).hexdigest()
    fx = load("plumbing_7b_256.npz")
    assert sha == str(fx["input_sha256"]), "regenerated inputs differ from the fixture's"
    return ts, fx
