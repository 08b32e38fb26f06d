"""Pin the float64 oracle against independent mathematics (CPU only).

Each check uses a different route to the same value than the oracle's own
formula: a matrix exponential, a sum-of-products (unrolled) form of the
recurrence, a closed form, a dual/quadratic form, autograd, or hand-built
known answers.  A plausible mistake in the oracle (dropped term, wrong sign,
index shift, swapped operand) fails at least one of them.
"""
import math

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import ssm_oracle as O

rng = np.random.default_rng(7)


# ------------------------------------------------------------------ ZOH
def test_zoh_matches_matrix_exponential():
    # textbook ZOH: expm([[a, b], [0, 0]] * dt) = [[exp(a dt), (exp(a dt)-1)/a * b], [0, 1]]
    H = 6
    A_log = rng.uniform(np.log(0.3), np.log(8.0), H)
    B = rng.normal(size=(1, 3, H))
    dt = rng.uniform(1e-4, 2.0, size=(1, 3))
    Abar, Bbar = O.zoh_discretize(A_log, B, dt)
    for t in range(3):
        for h in range(H):
            a = -np.exp(A_log[h])
            E = scipy.linalg.expm(np.array([[a, B[0, t, h]], [0.0, 0.0]]) * dt[0, t])
            assert Abar[0, t, h] == pytest.approx(E[0, 0], rel=1e-12)
            # oracle divides by (a + 1e-12), a perturbation of ~1e-12 relative
            assert Bbar[0, t, h] == pytest.approx(E[0, 1], rel=1e-10)


def test_zoh_limits():
    A_log = np.log(np.array([0.5, 2.0, 10.0]))
    B = np.ones((1, 2, 3))
    dt = np.array([[1e-9, 1e4]])
    Abar, Bbar = O.zoh_discretize(A_log, B, dt)
    a = -np.exp(A_log)
    np.testing.assert_allclose(Abar[0, 0], 1.0, rtol=1e-8)          # dt -> 0: Abar -> 1
    np.testing.assert_allclose(Bbar[0, 0], 1e-9, rtol=1e-6)         # Bbar -> dt*B
    np.testing.assert_allclose(Abar[0, 1], 0.0, atol=1e-300)        # dt*a -> -inf: Abar -> 0
    np.testing.assert_allclose(Bbar[0, 1], -1.0 / a, rtol=1e-9)     # Bbar -> -B/a


def test_reference_expm1_branch_is_taylor_below_threshold():
    x = np.array([-1e-6, 3e-6, -2e-3, 0.5])
    ref = O.expm1(x, "reference")
    np.testing.assert_allclose(ref[:2], x[:2] + x[:2] ** 2 / 2, rtol=0, atol=0)
    np.testing.assert_allclose(ref[2:], np.exp(x[2:]) - 1.0, rtol=0, atol=0)
    # and it deviates from exact expm1 by ~1e-13 relative near the threshold * eps64
    np.testing.assert_allclose(ref, np.expm1(x), rtol=1e-10)


# ------------------------------------------------------------------ elementwise scan
def _unrolled(u, A, B):
    """h_t = sum_{s<=t} (prod_{r=s+1..t} A_r) B_s u_s  -- explicit double loop."""
    Bsz, L, H = u.shape
    h = np.zeros_like(u)
    for t in range(L):
        acc = np.zeros((Bsz, H))
        for s in range(t + 1):
            prod = np.ones((Bsz, H))
            for r in range(s + 1, t + 1):
                prod = prod * A[:, r]
            acc += prod * B[:, s] * u[:, s]
        h[:, t] = acc
    return h


def test_ssm_forward_matches_unrolled_sum():
    Bsz, L, H = 2, 9, 3
    u, B, C = (rng.normal(size=(Bsz, L, H)) for _ in range(3))
    A = rng.uniform(0.2, 1.1, size=(Bsz, L, H))
    D = rng.normal(size=H)
    y, h = O.ssm_forward(u, A, B, C, D, BLK=4)
    h_ref = _unrolled(u, A, B)
    np.testing.assert_allclose(h, h_ref, rtol=1e-12)
    np.testing.assert_allclose(y, C * h_ref + D * u, rtol=1e-12)


def test_ssm_constant_coefficient_closed_form():
    L, a, b = 50, 0.93, 0.4
    u = np.ones((1, L, 1))
    A = np.full((1, L, 1), a)
    B = np.full((1, L, 1), b)
    _, h = O.ssm_forward(u, A, B, np.ones_like(u), np.zeros(1))
    t = np.arange(L)
    np.testing.assert_allclose(h[0, :, 0], b * (1 - a ** (t + 1)) / (1 - a), rtol=1e-12)


def test_ssm_prefix_sum_and_memoryless_cases():
    u = rng.normal(size=(2, 17, 4))
    one = np.ones_like(u)
    _, h = O.ssm_forward(u, one, one, one, np.zeros(4))
    np.testing.assert_allclose(h, np.cumsum(u, axis=1), rtol=1e-12)
    B = rng.normal(size=u.shape)
    _, h0 = O.ssm_forward(u, np.zeros_like(u), B, one, np.zeros(4))
    np.testing.assert_allclose(h0, B * u, rtol=0)


@pytest.mark.parametrize("BLK", [1, 3, 7, 16, 64])
def test_phase_pipeline_chunk_invariant(BLK):
    Bsz, L, H = 2, 37, 5
    u, B, C = (rng.normal(size=(Bsz, L, H)) for _ in range(3))
    A = rng.uniform(0.3, 1.0, size=(Bsz, L, H))
    D = rng.normal(size=H)
    nblk = O.nxt_pow2(-(-L // BLK))
    la, lx, carry = O.ssm_fwd_local(u, A, B, BLK, nblk)
    carry = O.ssm_carry_scan(carry, Bsz * H, nblk)
    h = O.ssm_fwd_apply(la, lx, carry, BLK, nblk)
    y = O.ssm_output(h, C, D, u)
    y_ref, h_ref = O.ssm_forward(u, A, B, C, D)
    np.testing.assert_allclose(h, h_ref, rtol=1e-11, atol=1e-13)
    np.testing.assert_allclose(y, y_ref, rtol=1e-11, atol=1e-13)
    # loc_a is the in-chunk cumulative product (ssm_scan.py:36-45)
    for blk in range(-(-L // BLK)):
        sl = slice(blk * BLK, min(L, blk * BLK + BLK))
        np.testing.assert_allclose(la[:, sl], np.cumprod(A[:, sl], axis=1), rtol=1e-12)
    # padded chunks store the identity carry
    ca = carry[: Bsz * H * nblk].reshape(Bsz * H, nblk)
    real = -(-L // BLK)
    if nblk > real:
        np.testing.assert_allclose(ca[:, real:], np.broadcast_to(ca[:, real - 1:real], ca[:, real:].shape))


def test_backward_matches_autograd_minus_skip_term():
    Bsz, L, H = 2, 13, 3
    t = lambda *s: torch.tensor(rng.normal(size=s), dtype=torch.float64, requires_grad=True)  # noqa
    u, B, C = t(Bsz, L, H), t(Bsz, L, H), t(Bsz, L, H)
    A = torch.tensor(rng.uniform(0.3, 1.0, size=(Bsz, L, H)), requires_grad=True)
    D = t(H)
    hs, s = [], torch.zeros(Bsz, H, dtype=torch.float64)
    for i in range(L):
        s = A[:, i] * s + B[:, i] * u[:, i]
        hs.append(s)
    h = torch.stack(hs, 1)
    y = C * h + D * u
    dY = torch.tensor(rng.normal(size=(Bsz, L, H)))
    y.backward(dY)
    hd = h.detach().numpy()
    du, dA, dB, dC = O.ssm_backward(u.detach(), A.detach(), B.detach(), C.detach(), hd, dY)
    np.testing.assert_allclose(du + D.detach().numpy() * dY.numpy(), u.grad.numpy(), rtol=1e-10)
    np.testing.assert_allclose(dA, A.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dB, B.grad.numpy(), rtol=1e-10)
    np.testing.assert_allclose(dC, C.grad.numpy(), rtol=1e-10)
    # the phase pipeline gives the same dH for any chunking
    for BLK in (2, 5, 16):
        nblk = O.nxt_pow2(-(-L // BLK))
        la, ld, carry = O.ssm_bwd_local(A.detach(), C.detach(), dY, BLK, nblk)
        carry = O.ssm_bwd_carry_scan(carry, Bsz * H, nblk)
        g = O.ssm_bwd_apply(la, ld, carry, u.detach(), A.detach(), B.detach(), hd, dY, BLK, nblk)
        for got, ref in zip(g, (du, dA, dB, dC)):
            np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


# ------------------------------------------------------------------ multihead
def _mh_inputs(Bsz=2, L=11, nh=3, hd=4, seed=3):
    r = np.random.default_rng(seed)
    return dict(
        u=r.normal(size=(Bsz, L, nh * hd)), A_log=r.uniform(0, np.log(6), size=(nh, hd)),
        B=r.normal(size=(Bsz, L, nh, hd)), C=r.normal(size=(Bsz, L, nh, hd)),
        dt=r.uniform(0.01, 0.8, size=(Bsz, L, nh)), D=r.normal(size=nh * hd))


def test_multihead_equals_elementwise_scan_after_lane_mapping():
    d = _mh_inputs()
    Bsz, L, nh, hd = d["B"].shape
    for disc in ("euler", "zoh"):
        y, hl = O.multihead_forward(d["u"], d["A_log"], d["B"], d["C"], d["dt"], d["D"], disc=disc)
        a = -np.exp(d["A_log"])
        Abar = np.exp(d["dt"][..., None] * a)
        coef = d["dt"][..., None] if disc == "euler" else np.expm1(d["dt"][..., None] * a) / a
        uu = d["u"].reshape(Bsz, L, nh, hd)
        flat = lambda x: x.reshape(Bsz, L, nh * hd)  # noqa: E731
        _, h = O.ssm_forward(flat(uu), flat(Abar), flat(coef * d["B"]), flat(d["C"]),
                             np.zeros(nh * hd))
        yh = (d["C"] * h.reshape(Bsz, L, nh, hd)).sum(-1) + (uu * d["D"].reshape(nh, hd)).sum(-1)
        np.testing.assert_allclose(y, np.repeat(yh, hd, axis=-1), rtol=1e-11, atol=1e-12)
        np.testing.assert_allclose(hl, h[:, -1].reshape(Bsz, nh, hd), rtol=1e-12)


def test_multihead_phases_match_fused_and_broadcast():
    d = _mh_inputs(L=19)
    Bsz, L, nh, hd = d["B"].shape
    for BLK in (1, 4, 8, 32):
        nblk = O.nxt_pow2(-(-L // BLK))
        la, lx, carry = O.multihead_fwd_local(d["u"], d["A_log"], d["B"], d["C"], d["dt"], nh, hd, BLK, nblk)
        carry = O.multihead_carry_scan(carry, Bsz * nh * hd, nblk)
        y = O.multihead_output(la, lx, carry, d["C"], d["D"], d["u"], nh, hd, BLK, nblk)
        y_ref, _ = O.multihead_forward(d["u"], d["A_log"], d["B"], d["C"], d["dt"], d["D"])
        np.testing.assert_allclose(y, y_ref, rtol=1e-11, atol=1e-12)
        yh = y.reshape(Bsz, L, nh, hd)
        assert np.all(yh == yh[..., :1])  # every slot of a head holds the same value


def test_multihead_phase_layout_known_answer():
    """Hand-computed phase intermediates at Bsz=1, nh=2, hd=2, BLK_L=2, L=4
    (NBLK=2), Euler, dt=1, B=C=1, D=0.  Lane (h, p) has decay 1/k with
    k = 2, 4, 8, 16 (A_log = log ln k) and input u[t, ch] = 1 + ch + 4t, so
    every value is a dyadic rational (exp(-ln k) = 1/k up to rounding, hence
    the 1e-13 bar).  The carry layout is
    [2, rows, NBLK] with row_flat = b*nh*hd + h*hd + p
    (multihead_ssm_kernel.py:98-100): a swapped (blk, row) order, a head/lane
    transposition or an inclusive/exclusive mix-up moves these numbers."""
    k = np.array([[2.0, 4.0], [8.0, 16.0]])
    A_log = np.log(np.log(k))
    u = (1.0 + np.arange(4)[None, :] + 4.0 * np.arange(4)[:, None])[None]    # [1,4,4]
    B = np.ones((1, 4, 2, 2))
    C = np.ones((1, 4, 2, 2))
    dt = np.ones((1, 4, 2))
    D = np.zeros(4)
    la, lx, carry = O.multihead_fwd_local(u, A_log, B, C, dt, 2, 2, 2, 2)
    A = np.array([0.5, 0.25, 0.125, 0.0625])                 # decay of rows 0..3
    # loc_a: in-chunk cumulative products, chunk 0 = steps 0-1, chunk 1 = steps 2-3
    np.testing.assert_allclose(la.reshape(4, 4), np.stack([A, A * A, A, A * A]), rtol=1e-13)
    # loc_x: in-chunk states from zero
    lx_ref = np.array([[1.0, 2.0, 3.0, 4.0],
                       [5.5, 6.5, 7.375, 8.25],
                       [9.0, 10.0, 11.0, 12.0],
                       [13.5 + 4.0, 16.5, 16.375, 16.75]])
    np.testing.assert_allclose(lx.reshape(4, 4), lx_ref, rtol=1e-13)
    # carry[row*NBLK + blk] (a part), carry[rows*NBLK + row*NBLK + blk] (x part)
    carry_ref = np.array([0.25, 0.25, 1 / 16, 1 / 16, 1 / 64, 1 / 64, 1 / 256, 1 / 256,
                          5.5, 17.5, 6.5, 16.5, 7.375, 16.375, 8.25, 16.75])
    np.testing.assert_allclose(carry, carry_ref, rtol=1e-13)
    # inclusive carry scan over the chunks of each row: block 1 = block 0 o block 1
    scanned = O.multihead_carry_scan(carry, 4, 2)
    scanned_ref = np.array([0.25, 1 / 16, 1 / 16, 1 / 256, 1 / 64, 1 / 4096, 1 / 256, 1 / 65536,
                            5.5, 18.875, 6.5, 16.90625, 7.375, 16.490234375, 8.25, 16.7822265625])
    np.testing.assert_allclose(scanned, scanned_ref, rtol=1e-13)
    # readout: y_head = sum_p h, stored to both slots of the head
    y = O.multihead_output(la, lx, scanned, C, D, u, 2, 2, 2, 2)
    yh = np.array([[3.0, 7.0], [12.0, 15.625], [23.375, 24.4375], [35.78125, 33.2724609375]])
    np.testing.assert_allclose(y[0], np.repeat(yh, 2, axis=1), rtol=1e-13)


def test_multihead_split_resume():
    d = _mh_inputs(L=20)
    cut = 7
    y, h = O.multihead_forward(d["u"], d["A_log"], d["B"], d["C"], d["dt"], d["D"], disc="zoh")
    part = lambda x, s: x[:, s]  # noqa: E731
    y1, h1 = O.multihead_forward(*(part(d[k], slice(0, cut)) for k in ("u",)), d["A_log"],
                                 d["B"][:, :cut], d["C"][:, :cut], d["dt"][:, :cut], d["D"], disc="zoh")
    y2, h2 = O.multihead_forward(d["u"][:, cut:], d["A_log"], d["B"][:, cut:], d["C"][:, cut:],
                                 d["dt"][:, cut:], d["D"], disc="zoh", h0=h1)
    np.testing.assert_allclose(np.concatenate([y1, y2], 1), y, rtol=1e-12)
    np.testing.assert_allclose(h2, h, rtol=1e-12)


# ------------------------------------------------------------------ Mamba-1 / SSD dual forms
def test_selective_scan_dual_form():
    r = np.random.default_rng(11)
    Bsz, L, Dc, N = 2, 12, 3, 4
    x = r.normal(size=(Bsz, L, Dc))
    dt = r.uniform(0.01, 0.3, size=(Bsz, L))
    A_log = r.uniform(np.log(0.5), np.log(5), size=(Dc, N))
    B, C = r.normal(size=(Bsz, L, N)), r.normal(size=(Bsz, L, N))
    D = r.normal(size=Dc)
    y, h = O.selective_scan(x, dt, A_log, B, C, D)
    a = -np.exp(A_log)                                                  # [Dc, N]
    cum = np.cumsum(dt, axis=1)                                         # [Bsz, L]
    y_ref = np.zeros_like(y)
    for t in range(L):
        for s in range(t + 1):
            decay = np.exp((cum[:, t] - cum[:, s])[:, None, None] * a)  # exp(a * sum dt_{s+1..t})
            bbar = np.expm1(dt[:, s][:, None, None] * a) / a * B[:, s][:, None, :]
            y_ref[:, t] += (C[:, t][:, None, :] * decay * bbar).sum(-1) * x[:, s]
    y_ref += D * x
    np.testing.assert_allclose(y, y_ref, rtol=1e-10, atol=1e-12)


def test_ssd_dual_form_and_stream_steps():
    r = np.random.default_rng(12)
    Bsz, L, H, P, N = 2, 10, 2, 3, 4
    x = r.normal(size=(Bsz, L, H, P))
    dt = r.uniform(0.01, 0.5, size=(Bsz, L, H))
    A_log = r.uniform(0, np.log(16), size=H)
    B, C = r.normal(size=(Bsz, L, H, N)), r.normal(size=(Bsz, L, H, N))
    D = r.normal(size=(H, P))
    y, hl = O.ssd_scan(x, dt, A_log, B, C, D)
    a = -np.exp(A_log)
    cum = np.cumsum(dt, axis=1)                                         # [Bsz, L, H]
    y_ref = np.zeros_like(y)
    for b in range(Bsz):
        for h in range(H):
            # Mamba-2 dual form: y = (Lmask o (C B^T)) x with segment decays
            Lm = np.zeros((L, L))
            for t in range(L):
                for s in range(t + 1):
                    Lm[t, s] = np.exp(a[h] * (cum[b, t, h] - cum[b, s, h])) * \
                        np.expm1(a[h] * dt[b, s, h]) / a[h]
            G = C[b, :, h] @ B[b, :, h].T                                # [L, L]
            y_ref[b, :, h] = (Lm * G) @ x[b, :, h] + D[h] * x[b, :, h]
    np.testing.assert_allclose(y, y_ref, rtol=1e-10, atol=1e-12)
    # k streaming steps == the scan
    state = np.zeros((Bsz, H, P, N))
    for t in range(L):
        ys = O.ssd_stream_step(x[:, t], dt[:, t], A_log, B[:, t], C[:, t], D, state)
        np.testing.assert_allclose(ys, y[:, t], rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(state, hl, rtol=1e-12)


# ------------------------------------------------------------------ interpolation
def _interp_case(V, M, tau, K=10, FTILE=128):
    V = np.asarray(V, float)[None]
    M = np.asarray(M, float)[None]
    tau = np.asarray(tau, float)[None]
    return O.time_aware_interp(V, M, tau, K, FTILE)[0]


def test_interp_fully_observed_interior_boundaries_and_affine():
    T, F = 6, 4
    tau = np.array([0.0, 0.5, 1.7, 2.0, 3.9, 4.0])
    V = np.arange(T * F, dtype=float).reshape(T, F)
    out = _interp_case(V, np.ones((T, F)), tau, FTILE=4)
    np.testing.assert_allclose(out[0], V[1])                 # t=0: only next -> V[1]
    np.testing.assert_allclose(out[-1], V[-2])               # t=T-1: only prev -> V[T-2]
    for t in range(1, T - 1):                                 # both neighbours -> time-weighted
        w = (tau[t] - tau[t - 1]) / (tau[t + 1] - tau[t - 1])
        np.testing.assert_allclose(out[t], (1 - w) * V[t - 1] + w * V[t + 1])
    Va = 3.0 + 2.0 * tau[:, None] * np.ones((1, F))           # affine in tau -> unchanged inside
    outa = _interp_case(Va, np.ones((T, F)), tau, FTILE=4)
    np.testing.assert_allclose(outa[1:-1], Va[1:-1], rtol=1e-12)


def test_interp_nearest_observed_tile_and_window():
    T, F = 12, 2
    tau = np.arange(T, dtype=float)
    V = 10.0 * np.arange(T)[:, None] + np.array([0.0, 1.0])
    M = np.zeros((T, F))
    M[2, 1] = 1.0     # one lane observed at t=2 -> the whole 2-lane tile counts
    M[9, 0] = 1.0
    out = _interp_case(V, M, tau, K=10, FTILE=2)
    # t=5: prev = 2 (nearest observed tile), next = 9 -> w = 3/7, using lane values there
    w = 3.0 / 7.0
    np.testing.assert_allclose(out[5], (1 - w) * V[2] + w * V[9])
    # t=2 is itself observed but neighbours exist (prev none within, next 9) -> V[9]
    np.testing.assert_allclose(out[2], V[9])
    # K=2: t=5 has no observed tile within 2 steps -> keeps its own value
    out2 = _interp_case(V, M, tau, K=2, FTILE=2)
    np.testing.assert_allclose(out2[5], V[5])
    np.testing.assert_allclose(out2[11], V[9])      # only prev (9) within 2
    np.testing.assert_allclose(out2[0], V[2])       # only next (2) within 2


def test_interp_tile_aggregate_is_per_tile_and_equal_times_give_half():
    T, F = 3, 4
    V = np.array([[1.0, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]])
    M = np.array([[1.0, 0, 0, 0], [0, 0, 0, 0], [0, 0, 0, 1]])
    tau = np.array([0.0, 1.0, 2.0])
    out = _interp_case(V, M, tau, FTILE=2)
    # tile 0 (lanes 0,1): only t=0 observed -> t=1 has prev only -> V[0]; tile 1: next only -> V[2]
    np.testing.assert_allclose(out[1], [1.0, 2.0, 11.0, 12.0])
    # equal timestamps: denominator 0 -> w = 0.5
    out_eq = _interp_case(np.array([[0.0], [7.0], [2.0]]), np.ones((3, 1)),
                          np.array([1.0, 1.0, 1.0]), FTILE=1)
    assert out_eq[1, 0] == pytest.approx(1.0)


def test_interp_step_and_fused_sequence_consistent():
    r = np.random.default_rng(5)
    Bsz, T, F = 2, 9, 5
    V = r.normal(size=(Bsz, T, F))
    M = (r.random((Bsz, T, F)) < 0.4).astype(float)
    tau = np.sort(r.uniform(0, 10, size=(Bsz, T)), axis=1)
    full = O.time_aware_interp(V, M, tau, K=3, FTILE=2)
    Ab, Bb = r.uniform(0.2, 0.9, F), r.normal(size=F)
    h = r.normal(size=(Bsz, F))
    for t in range(T):
        v, h_new = O.interp_ssm_step(V, M, tau, Ab, Bb, h, t, K=3, FTILE=2)
        np.testing.assert_allclose(v, full[:, t])
        np.testing.assert_allclose(h_new, Ab * h + Bb * full[:, t])
        h = h_new


# ------------------------------------------------------------------ streaming
def test_streaming_steps_equal_elementwise_scan():
    r = np.random.default_rng(8)
    Bsz, L, H = 3, 7, 5
    u, C = r.normal(size=(Bsz, L, H)), r.normal(size=(Bsz, L, H))
    Ab = r.uniform(0.1, 1.0, size=H)
    Bb = r.normal(size=H)
    D = r.normal(size=H)
    y_ref, h_ref = O.ssm_forward(u, np.broadcast_to(Ab, u.shape), np.broadcast_to(Bb, u.shape), C, D)
    h = np.zeros((Bsz, H))
    for t in range(L):
        h, y = O.streaming_step(u[:, t], h, Ab, Bb, C[:, t], D)
        np.testing.assert_allclose(y, y_ref[:, t], rtol=1e-12)
    np.testing.assert_allclose(h, h_ref[:, -1], rtol=1e-12)


def test_streaming_ring_known_answers():
    KR, H = 4, 4
    ring_V = np.zeros((1, KR, H))
    ring_M = np.zeros((1, KR, H))
    ring_tau = np.zeros((1, KR))
    head = np.array([0])
    ones = np.ones(H)
    z = np.zeros(H)
    # step 1: observed tile 0 only (lanes 0,1), value 5
    v1 = np.array([[5.0, 5.0, 0.0, 0.0]])
    m1 = np.array([[1.0, 0.0, 0.0, 0.0]])
    rV, rM, rt, hd, h, y = O.streaming_interp_step(ring_V, ring_M, ring_tau, head, v1, m1,
                                                   np.array([1.0]), np.zeros((1, H)), ones, ones,
                                                   ones[None], z, BLOCK_H=2, KRING=KR)
    assert hd[0] == 1 and rt[0, 1] == 1.0
    np.testing.assert_allclose(y[0], [5.0, 5.0, 0.0, 0.0])      # nothing to fill from
    # step 2: nothing observed -> tile 0 forward-fills from slot 1, tile 1 has no source
    v2 = np.array([[9.0, 9.0, 9.0, 9.0]])
    m2 = np.zeros((1, H))
    rV, rM, rt, hd, h2, y2 = O.streaming_interp_step(rV, rM, rt, hd, v2, m2, np.array([2.0]),
                                                     h, ones, ones, ones[None], z, BLOCK_H=2,
                                                     KRING=KR)
    assert hd[0] == 2
    np.testing.assert_allclose(h2[0], h[0] + np.array([5.0, 5.0, 9.0, 9.0]))


# ------------------------------------------------------------------ bwd / dt projection
def test_zoh_bwd_matches_autograd():
    r = np.random.default_rng(9)
    Bsz, T, H = 2, 5, 4
    A_log = torch.tensor(r.uniform(np.log(0.5), np.log(5), H), requires_grad=True)
    B = torch.tensor(r.normal(size=(Bsz, T, H)), requires_grad=True)
    dt = torch.tensor(r.uniform(0.01, 0.5, size=(Bsz, T)), requires_grad=True)
    a = -torch.exp(A_log)
    Abar = torch.exp(dt[..., None] * a)
    Bbar = torch.expm1(dt[..., None] * a) / (a + 1e-12) * B
    gA, gB = torch.tensor(r.normal(size=(Bsz, T, H))), torch.tensor(r.normal(size=(Bsz, T, H)))
    (Abar * gA + Bbar * gB).sum().backward()
    dA, dB, ddt = O.zoh_discretize_bwd(A_log.detach(), B.detach(), dt.detach(), Abar.detach(), gA, gB)
    np.testing.assert_allclose(dB, B.grad.numpy(), rtol=1e-9)
    np.testing.assert_allclose(ddt, dt.grad.numpy(), rtol=1e-9)
    np.testing.assert_allclose(dA, A_log.grad.numpy(), rtol=1e-7)


def test_dt_projection_matches_torch_softplus():
    r = np.random.default_rng(10)
    raw, W, bias = r.normal(size=(2, 3, 4)) * 3, r.normal(size=(4, 5)) * 4, r.normal(size=5)
    out = O.dt_project_softplus(raw, W, bias, 1e-3, 0.5)
    acc = torch.tensor(raw) @ torch.tensor(W) + torch.tensor(bias)
    ref = torch.nn.functional.softplus(acc).clamp(1e-3, 0.5).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-12)
    assert math.isclose(float(O.dt_project_softplus(np.array([[[100.0]]]), np.array([[1.0]]),
                                                    np.zeros(1), 0.0, 50.0)[0, 0, 0]), 50.0)
