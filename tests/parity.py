"""Shared parity helpers for the test suite.

Tolerances are derived from fp32 rounding error bounds, not fitted: for a
dot product of K terms in any summation order, |computed - exact| <=
gamma_K * sum|terms| with gamma_K ~ K * 2^-24.  Two implementations that
both satisfy the bound differ by at most twice it.
"""
import numpy as np

EPS32 = 2.0 ** -24


def dot_bound(absA, absB, K):
    """Per-output bound 2*gamma_K*sum_k |A_k||B_kn| for C = A @ B."""
    return 2.0 * K * EPS32 * (absA @ absB)


def assert_close_bound(got, ref, bound, slack=1e-6, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    lim = np.asarray(bound, np.float64) + slack * (1.0 + np.abs(ref))
    bad = err > lim
    if bad.any():
        i = int(np.flatnonzero(bad.ravel())[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} outside the bound; first at {i}: "
            f"got {got.ravel()[i]!r} ref {ref.ravel()[i]!r} err {err.ravel()[i]:.3e} lim {lim.ravel()[i]:.3e}")


TIE_TOL = 1e-4  # largest oracle top-2 logit gap at which the greedy ids may part

# One line per full-depth run (configuration, path, how many free-running
# greedy ids agreed with the oracle's, teacher-forced agreement, logit
# error), printed in pytest's terminal summary even under -q.
IDENTITY_RECORDS = []


def greedy_agree(gpu_ids, ref_ids, ref_top2, tie_tol=TIE_TOL):
    """Greedy sequences must be identical, except that they may part at a
    step where the reference's own top-2 logit gap is below tie_tol (a near
    tie that summation order legitimately decides); after a parting the
    contexts differ, so the comparison of the free-running sequences ends
    there (the teacher-forced checks cover the later steps).  Returns the
    number of leading tokens that agree; prints any parting."""
    gpu_ids = np.asarray(gpu_ids)
    ref_ids = np.asarray(ref_ids)
    n = min(len(gpu_ids), len(ref_ids))
    for k in range(n):
        if gpu_ids[k] != ref_ids[k]:
            gap = float(ref_top2[k, 0] - ref_top2[k, 1])
            print(f"[parity] greedy ids part at step {k}: gpu {gpu_ids[k]} ref {ref_ids[k]}, "
                  f"reference top-2 gap {gap:.3e}", flush=True)
            assert gap < tie_tol, (
                f"greedy ids differ at step {k}: gpu {gpu_ids[k]} ref {ref_ids[k]} "
                f"with reference top-2 gap {gap:.3e} >= {tie_tol}")
            return k
    assert len(gpu_ids) == len(ref_ids), f"lengths differ: {len(gpu_ids)} vs {len(ref_ids)}"
    return n


def masked_first_max(logits, forbid_eos=True, eos=50256):
    """sample_next_token's greedy choice (main.c:1882-1903): EOS masked,
    first maximum."""
    lg = np.array(logits, np.float32, copy=True)
    if forbid_eos and eos < lg.size:
        lg[eos] = -1e30
    return int(np.argmax(lg))


def random_prompt(n, vocab, seed):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.int32)
