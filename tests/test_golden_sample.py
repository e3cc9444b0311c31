"""oracle.sample against the reference's own sample() (tokenrush/sample.py:30-51), as recorded in
tests/golden/sample_vectors.npz by tests/golden/make_sample_vectors.py (the reference run with
torch on the CPU; inputs regenerated here from seeds, checked by SHA-256).

* Rows whose 65 largest logits are distinct bf16 values (248320-wide rows and 20480 draws over
  512-wide rows, 8 parameter sets including greedy, top_k 1 and top_p 0.5): every token equals the
  reference's, so the oracle's fixed-order fp32 softmax / cumsum (and the texp exponential) pick
  what torch's CPU softmax / cumsum pick on these inputs.
* Rows with bf16 ties among their top 64 (plain N(0, 2) logits at V = 248320): torch.topk orders
  equal values arbitrarily (sample.py:37-38 says so), the oracle by ascending index. There the
  tokens may differ, but only inside a tie: the two picks always carry the same logit value, and
  greedy rows (temperature 0, argmax by first index) are equal."""
import os
import sys

import numpy as np
import pytest

from oracle import accept as oa

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import sample_cases as sc  # noqa: E402

VEC = np.load(os.path.join(HERE, "golden", "sample_vectors.npz"))


def _group(name):
    bits, u = sc.group_inputs(name)
    assert sc.digest(bits) == str(VEC[name + "_logits_sha256"]) and sc.digest(u) == str(VEC[name + "_u_sha256"])
    return sc.bits_to_f32(bits), u, VEC[name + "_tokens"]


def test_params_match_fixture():
    assert np.array_equal(VEC["params"], np.array(sc.PARAMS, np.float64))


@pytest.mark.parametrize("name", ["full_vocab", "small_vocab"])
def test_tie_free_rows_match_reference_bit_exact(name):
    lg, u, want = _group(name)
    for pi, (T, top_p, top_k) in enumerate(sc.PARAMS):
        for d in range(u.shape[2]):
            got = oa.sample(lg, T, top_p, top_k, u[:, pi, d])
            assert np.array_equal(got, want[:, pi, d]), (name, sc.PARAMS[pi], d)


def test_tied_rows_differ_only_inside_ties():
    lg, u, want = _group("tied")
    differ = 0
    for pi, (T, top_p, top_k) in enumerate(sc.PARAMS):
        for d in range(u.shape[2]):
            got = oa.sample(lg, T, top_p, top_k, u[:, pi, d])
            rows = np.arange(lg.shape[0])
            assert np.array_equal(lg[rows, got], lg[rows, want[:, pi, d]]), (sc.PARAMS[pi], d)
            if T == 0:
                assert np.array_equal(got, want[:, pi, d])
            differ += int((got != want[:, pi, d]).sum())
    print(f"tied rows: {differ} of {want.size} tokens differ (same logit value each time)")
