"""Property tests of the float64 oracle over random shapes and values
(hypothesis): invariants every scan on the path must satisfy, independent of
how the oracle computes it -- linearity in the input, causality, split/resume
through h0/h_last, and for the interpolation invariance under an affine change
of the time axis and idempotence on fully observed data.  A wrong index, a
dropped term or a transposed operand in a restatement breaks at least one."""
import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from oracle import ssm_oracle as O

SET = settings(max_examples=25, deadline=None, suppress_health_check=[HealthCheck.too_slow])


def _rng(seed):
    return np.random.default_rng(seed)


def _close(a, b, tol=1e-10):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    scale = max(1.0, float(np.max(np.abs(b))) if b.size else 1.0)
    assert np.max(np.abs(a - b)) <= tol * scale if a.size else True


def _selective(seed, Bsz, L, Dc, N, shared_dt):
    r = _rng(seed)
    x = r.standard_normal((Bsz, L, Dc))
    dt = r.exponential(0.3, (Bsz, L) if shared_dt else (Bsz, L, Dc))
    A_log = r.uniform(np.log(0.5), np.log(5.0), (Dc, N))
    B = r.standard_normal((Bsz, L, N)) / np.sqrt(N)
    C = r.standard_normal((Bsz, L, N)) / np.sqrt(N)
    D = r.standard_normal(Dc)
    return x, dt, A_log, B, C, D


def _ssd(seed, Bsz, L, H, P, N):
    r = _rng(seed)
    x = r.standard_normal((Bsz, L, H, P))
    dt = r.exponential(0.3, (Bsz, L, H))
    A_log = r.uniform(0.0, np.log(8.0), H)
    B = r.standard_normal((Bsz, L, H, N)) / np.sqrt(N)
    C = r.standard_normal((Bsz, L, H, N)) / np.sqrt(N)
    D = r.standard_normal((H, P))
    return x, dt, A_log, B, C, D


def _multihead(seed, Bsz, L, nh, hd):
    r = _rng(seed)
    u = r.standard_normal((Bsz, L, nh * hd))
    A_log = r.uniform(0.0, np.log(8.0), (nh, hd))
    B = r.standard_normal((Bsz, L, nh, hd)) / np.sqrt(hd)
    C = r.standard_normal((Bsz, L, nh, hd)) / np.sqrt(hd)
    dt = r.exponential(0.3, (Bsz, L, nh))
    D = r.standard_normal(nh * hd)
    return u, A_log, B, C, dt, D


shapes = st.tuples(st.integers(1, 2), st.integers(1, 24), st.integers(1, 5), st.integers(1, 6))


@SET
@given(seed=st.integers(0, 2**31 - 1), shp=shapes, shared=st.booleans(),
       disc=st.sampled_from(["zoh", "euler"]), al=st.floats(-2, 2), be=st.floats(-2, 2))
def test_selective_scan_linear_in_x_and_h0(seed, shp, shared, disc, al, be):
    """y and h_last are linear in (x, h0) jointly for fixed dt, A, B, C, D."""
    Bsz, L, Dc, N = shp
    x1, dt, A_log, B, C, D = _selective(seed, Bsz, L, Dc, N, shared)
    r = _rng(seed + 1)
    x2 = r.standard_normal(x1.shape)
    h1, h2 = r.standard_normal((Bsz, Dc, N)), r.standard_normal((Bsz, Dc, N))
    y1, s1 = O.selective_scan(x1, dt, A_log, B, C, D, h0=h1, disc=disc)
    y2, s2 = O.selective_scan(x2, dt, A_log, B, C, D, h0=h2, disc=disc)
    y, s = O.selective_scan(al * x1 + be * x2, dt, A_log, B, C, D, h0=al * h1 + be * h2, disc=disc)
    _close(y, al * y1 + be * y2, 1e-9)
    _close(s, al * s1 + be * s2, 1e-9)


@SET
@given(seed=st.integers(0, 2**31 - 1), shp=shapes, cut=st.integers(0, 24),
       disc=st.sampled_from(["zoh", "euler"]))
def test_selective_scan_causal_and_split_resume(seed, shp, cut, disc):
    """Outputs before t ignore every input at or after t; the scan of a
    sequence equals the scan of its tail started from the head's h_last."""
    Bsz, L, Dc, N = shp
    cut = min(cut, L)
    x, dt, A_log, B, C, D = _selective(seed, Bsz, L, Dc, N, False)
    y, s = O.selective_scan(x, dt, A_log, B, C, D, disc=disc)
    xp = x.copy()
    xp[:, cut:] += 7.0
    yp, _ = O.selective_scan(xp, dt, A_log, B, C, D, disc=disc)
    _close(yp[:, :cut], y[:, :cut], 0)
    ya, sa = O.selective_scan(x[:, :cut], dt[:, :cut], A_log, B[:, :cut], C[:, :cut], D, disc=disc)
    yb, sb = O.selective_scan(x[:, cut:], dt[:, cut:], A_log, B[:, cut:], C[:, cut:], D, h0=sa,
                              disc=disc)
    _close(np.concatenate([ya, yb], 1), y, 1e-12)
    _close(sb, s, 1e-12)


@SET
@given(seed=st.integers(0, 2**31 - 1),
       shp=st.tuples(st.integers(1, 2), st.integers(1, 20), st.integers(1, 3), st.integers(1, 5),
                     st.integers(1, 5)),
       cut=st.integers(0, 20), disc=st.sampled_from(["zoh", "euler"]), al=st.floats(-2, 2))
def test_ssd_scan_split_resume_and_linearity(seed, shp, cut, disc, al):
    Bsz, L, H, P, N = shp
    cut = min(cut, L)
    x, dt, A_log, B, C, D = _ssd(seed, Bsz, L, H, P, N)
    y, s = O.ssd_scan(x, dt, A_log, B, C, D, disc=disc)
    ya, sa = O.ssd_scan(x[:, :cut], dt[:, :cut], A_log, B[:, :cut], C[:, :cut], D, disc=disc)
    yb, sb = O.ssd_scan(x[:, cut:], dt[:, cut:], A_log, B[:, cut:], C[:, cut:], D, h0=sa, disc=disc)
    _close(np.concatenate([ya, yb], 1), y, 1e-12)
    _close(sb, s, 1e-12)
    y2, s2 = O.ssd_scan(al * x, dt, A_log, B, C, D, disc=disc)
    _close(y2, al * y, 1e-9)
    _close(s2, al * s, 1e-9)


@SET
@given(seed=st.integers(0, 2**31 - 1),
       shp=st.tuples(st.integers(1, 2), st.integers(1, 20), st.integers(1, 3), st.integers(1, 6)),
       cut=st.integers(0, 20), disc=st.sampled_from(["zoh", "euler"]))
def test_multihead_causal_and_split_resume(seed, shp, cut, disc):
    Bsz, L, nh, hd = shp
    cut = min(cut, L)
    u, A_log, B, C, dt, D = _multihead(seed, Bsz, L, nh, hd)
    y, s = O.multihead_forward(u, A_log, B, C, dt, D, disc=disc)
    up = u.copy()
    up[:, cut:] -= 3.0
    yp, _ = O.multihead_forward(up, A_log, B, C, dt, D, disc=disc)
    _close(yp[:, :cut], y[:, :cut], 0)
    ya, sa = O.multihead_forward(u[:, :cut], A_log, B[:, :cut], C[:, :cut], dt[:, :cut], D,
                                 disc=disc)
    yb, sb = O.multihead_forward(u[:, cut:], A_log, B[:, cut:], C[:, cut:], dt[:, cut:], D,
                                 h0=sa, disc=disc)
    _close(np.concatenate([ya, yb], 1), y, 1e-12)
    _close(sb, s, 1e-12)


@SET
@given(seed=st.integers(0, 2**31 - 1),
       shp=st.tuples(st.integers(1, 2), st.integers(1, 30), st.integers(1, 8)),
       K=st.integers(0, 6), ft=st.sampled_from([1, 2, 4, 8]), p=st.floats(0.0, 1.0),
       scale=st.floats(0.01, 100.0), shift=st.floats(-1e3, 1e3))
def test_interp_invariant_under_affine_time(seed, shp, K, ft, p, scale, shift):
    """The interpolation weights are ratios of time differences: the result is
    unchanged when tau becomes scale * tau + shift (scale > 0), for both the
    reference per-tile mode and the corrected per-feature mode."""
    Bsz, T, F = shp
    r = _rng(seed)
    tau = np.sort(r.uniform(0, 10, (Bsz, T)), 1)
    M = (r.random((Bsz, T, F)) < p).astype(np.float64)
    V = r.standard_normal((Bsz, T, F)) * M
    tau2 = scale * tau + shift
    _close(O.time_aware_interp(V, M, tau2, K, ft), O.time_aware_interp(V, M, tau, K, ft), 1e-7)
    _close(O.time_aware_interp_corrected(V, M, tau2, K), O.time_aware_interp_corrected(V, M, tau, K),
           1e-7)


@SET
@given(seed=st.integers(0, 2**31 - 1),
       shp=st.tuples(st.integers(1, 2), st.integers(1, 30), st.integers(1, 8)),
       K=st.integers(0, 6))
def test_corrected_interp_fixes_observed_and_is_idempotent(seed, shp, K):
    """Observed values are kept, and interpolating an already interpolated
    sequence with the same mask changes nothing (every filled value is a
    combination of observed ones, which are kept)."""
    Bsz, T, F = shp
    r = _rng(seed)
    tau = np.sort(r.uniform(0, 10, (Bsz, T)), 1)
    M = (r.random((Bsz, T, F)) < 0.5).astype(np.float64)
    V = r.standard_normal((Bsz, T, F))
    out = O.time_aware_interp_corrected(V, M, tau, K)
    obs = M > 0.5
    assert np.array_equal(out[obs], V[obs])
    _close(O.time_aware_interp_corrected(out, M, tau, K), out, 0)


@SET
@given(seed=st.integers(0, 2**31 - 1), rank=st.integers(1, 8), H=st.integers(1, 6),
       lo=st.floats(1e-4, 0.5), width=st.floats(0.0, 5.0))
def test_dt_projection_bounds_and_monotone_in_bias(seed, rank, H, lo, width):
    r = _rng(seed)
    raw = r.standard_normal((2, 5, rank))
    W = r.standard_normal((rank, H))
    bias = r.standard_normal(H)
    hi = lo + width
    dt = O.dt_project_softplus(raw, W, bias, lo, hi)
    assert np.all(dt >= lo) and np.all(dt <= hi)
    dt2 = O.dt_project_softplus(raw, W, bias + 0.5, lo, hi)
    assert np.all(dt2 >= dt)        # softplus and clamp are non-decreasing
    pre = np.einsum("btr,rh->bth", raw, W) + bias
    assert np.all(O.dt_project_softplus(raw, W, bias, 0.0, np.inf) >= np.maximum(pre, 0.0) - 1e-12)
