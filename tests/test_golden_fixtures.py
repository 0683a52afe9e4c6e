"""The committed golden fixtures are well formed and describe the workload they claim to."""
import os

import numpy as np

import q35

HERE = os.path.join(os.path.dirname(__file__), "golden")


def test_e2e_2b_fixture_shape_and_prompt():
    g = np.load(os.path.join(HERE, "e2e_2b_seed0.npz"))
    d = q35.dims_2b()
    prompt, toks, margins = g["prompt"], g["tokens"], g["margins"]
    assert int(g["seed"]) == 0
    assert prompt.shape == (512,) and toks.shape == (513,) and margins.shape == (513,)
    # the prompt is the one bench.py feeds: default_rng(seed).integers(0, vocab, 512)
    np.testing.assert_array_equal(prompt, np.random.default_rng(0).integers(0, d.vocab, 512).astype(np.int32))
    assert toks.min() >= 0 and toks.max() < d.vocab
    assert (margins >= 0).all()
