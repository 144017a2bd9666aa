"""Loading helpers for the committed golden fixtures under tests/golden/."""

import os
from functools import lru_cache

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@lru_cache(maxsize=None)
def load(name):
    return np.load(os.path.join(GOLDEN, name))  # plain arrays: allow_pickle stays False


def pywt_input(seed, shape):
    return np.random.RandomState(int(seed)).standard_normal(shape)


def cwt_compare(actual, g, key, rtol_max=1e-10):
    """Compare ``actual`` (..., N) (complex or real) with a fixture stored either in full or as
    head + random projections along time; tolerance relative to the fixture's max."""
    import torch
    a = actual.detach().cpu()
    if a.is_complex():
        a = torch.view_as_real(a).movedim(-1, -2)
    a = a.double().numpy()
    if key in g.files:
        ref = g[key]
        np.testing.assert_allclose(a, ref, rtol=0, atol=rtol_max * max(np.abs(ref).max(), 1e-300))
        return
    head, sk = g[key + "@head"], g[key + "@sketch"]
    n = a.shape[-1]
    vecs = np.random.RandomState(12345).standard_normal((n, sk.shape[-1]))
    np.testing.assert_allclose(a[..., :head.shape[-1]], head, rtol=0,
                               atol=rtol_max * max(np.abs(head).max(), 1e-300))
    scale = max(np.abs(sk).max(), 1e-300)
    np.testing.assert_allclose(a @ vecs, sk, rtol=0, atol=rtol_max * scale * 10)
