"""The float64 references the GPU tests compare against (tests/_synth.py),
checked on the CPU: x @ W_public formed two ways agree, and both agree with
the oracle's projection (prepare, inner, finish with the reference's f16
rounding points) within the 1e-3 bar."""
import numpy as np

from oracle import oracle as O
from tests import _synth as S


def test_public_matmul_matches_dense_public_weight():
    rng = np.random.default_rng(5)
    in_f, out_f, n = 384, 256, 48
    t, suh, svh = S.linear(rng, in_f, out_f, n)
    x = S.activations(rng, 7, in_f).astype(np.float64)
    w = O.reconstruct_inner(t, in_f, out_f, n)
    dense = x @ S.public_weight(w, suh, svh)
    fact = S.public_matmul(x, w, suh, svh)
    assert np.abs(dense - fact).max() <= 1e-12 * np.abs(dense).max()
    yo = S.h2f(O.project(x.astype(np.float32), t, suh, svh, in_f, out_f, n))
    assert S.rel_fro(yo, fact) < 1e-3
    assert S.row_rel(yo, fact).max() < 2e-3
    # a transposed weight (a plausible indexing mistake) fails the bar
    bad = S.public_matmul(x, w.reshape(out_f, in_f).T.copy().reshape(in_f, out_f), suh, svh)
    assert S.rel_fro(bad, fact) > 0.5
