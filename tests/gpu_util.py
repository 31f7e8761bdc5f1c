"""Helpers for the GPU parity tests (imported by tests/test_gpu_*.py)."""
import numpy as np

from wisp_amd import synth
from wisp_amd.hip import DeviceBuffer, to_device


def expert_rng(seed, e):
    return np.random.default_rng([seed, e])


def make_expert(seed, e, inter, hidden, gs, zeros=False, out=None):
    return synth.make_blob(expert_rng(seed, e), inter, hidden, gs, expert=e, zeros=zeros, out=out)


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def cosine(got, want):
    a = np.asarray(got, np.float64).ravel()
    b = np.asarray(want, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))


# Parity bar for fp16 outputs: max |err| / max |ref| <= 1e-2 and cosine
# >= 0.9999 against the CPU oracle.
MAX_REL = 1e-2
MIN_COS = 0.9999


def assert_close(got, want, what=""):
    if not np.any(np.asarray(want)):
        # nothing routed to this token: the output must be exactly zero
        assert not np.any(np.asarray(got)), f"{what}: expected all zeros"
        return 0.0, 1.0
    r, c = rel_err(got, want), cosine(got, want)
    assert r <= MAX_REL and c >= MIN_COS, f"{what}: max-rel-err {r:.3e}, cosine {c:.7f}"
    return r, c


def assert_valid_topk(keys, sel, k, tol, what=""):
    """A selection decided by a near-tie of float64 `keys` (NaN or -inf:
    never selectable) must still be a top-k within `tol`: k distinct experts
    (or every selectable one when fewer), each no more than tol below the
    k-th largest key, no unselected key more than tol above it, and keys
    non-increasing in rank order within tol."""
    keys = np.asarray(keys, np.float64)
    ok = np.isfinite(keys)
    sel = [int(e) for e in sel if e >= 0]
    n_ok = int(ok.sum())
    assert len(sel) == min(k, n_ok) and len(set(sel)) == len(sel), (what, sel)
    assert all(ok[e] for e in sel), (what, sel)
    if not sel:
        return
    kth = np.sort(keys[ok])[::-1][len(sel) - 1]
    assert np.all(keys[sel] >= kth - tol), (what, sel, keys[sel], kth)
    rest = np.setdiff1d(np.nonzero(ok)[0], sel)
    if rest.size:
        assert np.max(keys[rest]) <= kth + tol, (what, np.max(keys[rest]), kth)
    assert np.all(np.diff(keys[sel]) <= tol), (what, keys[sel])
