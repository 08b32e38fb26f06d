"""The opt-in corrected interpolation oracle (per-feature neighbours, observed
values kept) pinned by closed forms, by the reference-mode oracle where the
two must agree, and by a scalar brute force."""
import numpy as np

from oracle import ssm_oracle as O


def _inputs(Bsz=2, T=40, F=6, p=0.3, seed=0):
    rng = np.random.default_rng(seed)
    V = rng.normal(size=(Bsz, T, F))
    M = (rng.random((Bsz, T, F)) < p).astype(float)
    tau = np.sort(rng.random((Bsz, T)) * 20, axis=1)
    return V, M, tau


def test_observed_values_kept():
    V, M, tau = _inputs()
    out = O.time_aware_interp_corrected(V, M, tau, K=5)
    assert np.array_equal(out[M > 0.5], V[M > 0.5])


def test_affine_in_time_is_exact():
    """V = alpha + beta tau on every step: an unobserved entry with both
    neighbours is interpolated back onto the line exactly."""
    V, M, tau = _inputs(T=60, p=0.4, seed=1)
    alpha, beta = np.array([0.5, -1, 2, 0, 3, 1.5]), np.array([1, 2, -0.5, 0.25, 0, -3.0])
    V = alpha[None, None, :] + beta[None, None, :] * tau[:, :, None]
    K = 6
    out = O.time_aware_interp_corrected(V, M, tau, K=K)
    obs = M > 0.5
    Bsz, T, F = V.shape
    both = np.zeros_like(obs)
    for t in range(T):
        lo, hi = max(0, t - K), min(T, t + K + 1)
        both[:, t] = obs[:, lo:t].any(1) & obs[:, t + 1:hi].any(1)
    sel = both & ~obs
    assert sel.sum() > 50
    assert np.allclose(out[sel], V[sel], rtol=1e-12, atol=1e-12)


def test_one_sided_fills_and_no_neighbour():
    V = np.arange(10, dtype=float).reshape(1, 10, 1) * 10.0
    tau = np.arange(10, dtype=float).reshape(1, 10)
    M = np.zeros((1, 10, 1))
    M[0, 2, 0] = 1                                       # only step 2 observed
    out = O.time_aware_interp_corrected(V, M, tau, K=3)[0, :, 0]
    assert out[2] == 20.0                                 # kept
    assert list(out[3:6]) == [20.0, 20.0, 20.0]           # forward fill within K
    assert out[6] == 60.0                                 # beyond K: V itself
    assert list(out[0:2]) == [20.0, 20.0]                 # backward fill


def test_zero_window_is_identity():
    V, M, tau = _inputs()
    assert np.array_equal(O.time_aware_interp_corrected(V, M, tau, K=0), V)


def test_tile_uniform_masks_match_reference_on_unobserved_steps():
    """When every feature of a tile shares its mask, per-feature neighbours
    equal per-tile ones, so the two modes agree wherever the step is
    unobserved (observed steps: corrected keeps V, the reference may not)."""
    rng = np.random.default_rng(3)
    Bsz, T, F, FT = 2, 50, 8, 4
    V = rng.normal(size=(Bsz, T, F))
    tau = np.sort(rng.random((Bsz, T)) * 10, axis=1)
    mt = (rng.random((Bsz, T, F // FT)) < 0.3).astype(float)
    M = np.repeat(mt, FT, axis=2)
    ref = O.time_aware_interp(V, M, tau, K=5, FTILE=FT)
    cor = O.time_aware_interp_corrected(V, M, tau, K=5)
    un = M < 0.5
    assert np.allclose(cor[un], ref[un], rtol=0, atol=1e-12)
    assert np.array_equal(cor[~un], V[~un])


def test_brute_force_scalar_loops():
    V, M, tau = _inputs(Bsz=1, T=25, F=3, p=0.25, seed=4)
    K = 4
    out = O.time_aware_interp_corrected(V, M, tau, K=K)
    T, F = V.shape[1:]
    for t in range(T):
        for f in range(F):
            if M[0, t, f] > 0.5:
                want = V[0, t, f]
            else:
                p = next((t - k for k in range(1, K + 1) if t - k >= 0 and M[0, t - k, f] > 0.5), None)
                n = next((t + k for k in range(1, K + 1) if t + k < T and M[0, t + k, f] > 0.5), None)
                if p is not None and n is not None:
                    den = tau[0, n] - tau[0, p]
                    w = (tau[0, t] - tau[0, p]) / den if den > 1e-9 else 0.5
                    w = min(max(w, 0.0), 1.0)
                    want = (1 - w) * V[0, p, f] + w * V[0, n, f]
                elif p is not None:
                    want = V[0, p, f]
                elif n is not None:
                    want = V[0, n, f]
                else:
                    want = V[0, t, f]
            assert abs(out[0, t, f] - want) < 1e-12


def _ring_state(S, KR, H, seed):
    rng = np.random.default_rng(seed)
    return [np.zeros((S, KR, H)), np.zeros((S, KR, H)), np.zeros((S, KR)),
            np.zeros(S, dtype=np.int64), rng.normal(size=(S, H))]


def test_streaming_corrected_matches_reference_for_tile_uniform_masks():
    rng = np.random.default_rng(5)
    S, KR, H, BH = 3, 6, 8, 4
    st_r = _ring_state(S, KR, H, 6)
    st_c = [x.copy() for x in st_r]
    Ab, Bb, D = rng.random(H), rng.random(H), rng.random(H)
    for step in range(12):
        mt = (rng.random((S, H // BH)) < 0.3).astype(float)
        m = np.repeat(mt, BH, axis=1)
        v = rng.normal(size=(S, H)) * m
        tau = np.full(S, float(step))
        C = rng.normal(size=(S, H))
        r = O.streaming_interp_step(*st_r[:4], v, m, tau, st_r[4], Ab, Bb, C, D, BH, KR)
        c = O.streaming_interp_step_corrected(*st_c[:4], v, m, tau, st_c[4], Ab, Bb, C, D, KR)
        assert np.allclose(r[5], c[5], atol=1e-12) and np.array_equal(r[3], c[3])
        st_r, st_c = list(r[:5]), list(c[:5])


def test_streaming_corrected_per_feature_fill():
    S, KR, H = 1, 4, 3
    st = _ring_state(S, KR, H, 7)
    st[4] = np.zeros((S, H))
    Ab, Bb, C, D = np.zeros(H), np.ones(H), np.zeros((S, H)), np.ones(H)   # y = vhat
    seq = [(np.array([[1.0, 2.0, 3.0]]), np.array([[1.0, 0.0, 1.0]])),
           (np.array([[4.0, 5.0, 6.0]]), np.array([[0.0, 0.0, 1.0]])),
           (np.array([[7.0, 8.0, 9.0]]), np.array([[0.0, 1.0, 0.0]]))]
    ys = []
    for i, (v, m) in enumerate(seq):
        out = O.streaming_interp_step_corrected(*st[:4], v, m, np.array([float(i)]), st[4],
                                                Ab, Bb, C, D, KR)
        st = list(out[:5])
        ys.append(out[5][0])
    assert list(ys[0]) == [1.0, 2.0, 3.0]      # features 0, 2 observed; 1 has no history
    assert list(ys[1]) == [1.0, 5.0, 6.0]      # f0 filled from step 0, f1 no history, f2 kept
    assert list(ys[2]) == [1.0, 8.0, 6.0]      # f0 from step 0, f1 kept, f2 from step 1
