"""Pins of the float64 oracle (oracle/scan_oracle.c) on the CPU.

The reference holds no data files or golden vectors for the scan, so the
oracle is pinned by what the mathematics fixes (mamba_metal/scan.py:13-41):

* forward: an independent O(T^2) closed-form evaluation with no recurrence;
  T = 1, Aneg = 0 (prefix sum), constant inputs (geometric series), x = 0;
  linearity in x, causality, checkpoint = state at the chunk's last step,
  decode steps chained = the scan;
* backward: central finite differences of the oracle's own forward for every
  input (and for the returned state, dh_last), a directional (JVP/VJP)
  dot-product test, and the brute-force dC = sum_d dy * h;
* each check rejects a planted mistake (a transposed operand, a dropped term,
  a wrong sign), so a plausible slip in the oracle cannot pass it;
* the block's causal depthwise conv1d + SiLU (model.py:174-175, :244):
  numpy's full convolution with the reversed kernel, the pointwise K = 1
  case, causality, finite differences and the VJP dot product.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle

RNG_SEED = 20240


def _inputs(bt, t_len, d, n, seed, style="ref"):
    return [a.astype(np.float64) for a in oracle.make_inputs(bt, t_len, d, n, seed, style)]


def _h_all(x, dt, aneg, b_in, c_in):
    """Every state h[b,t,d,n] from the decode-step oracle chained over t."""
    bt, t_len, d = x.shape
    n = aneg.shape[1]
    h = np.zeros((bt, d, n))
    hs = []
    for t in range(t_len):
        h, _ = oracle.scan_step(h, x[:, t], dt[:, t], aneg, b_in[:, t], c_in[:, t])
        hs.append(h)
    return np.stack(hs, axis=1)


# ------------------------------------------------------------------ forward

@pytest.mark.parametrize("shape", [(2, 1, 3, 4), (1, 17, 5, 8), (2, 40, 7, 5), (1, 33, 4, 16)])
def test_forward_matches_the_closed_form(shape):
    arrs = _inputs(*shape, seed=RNG_SEED + shape[1])
    y, _, h_last = oracle.scan_fwd(*arrs)
    y_cf, h_cf = oracle.scan_fwd_closed_form(*arrs)
    assert np.abs(y - y_cf).max() <= 1e-12 * max(1.0, np.abs(y_cf).max())
    assert np.abs(h_last - h_cf).max() <= 1e-12 * max(1.0, np.abs(h_cf).max())


def test_single_step_is_dt_x_times_c_dot_b():
    x, dt, aneg, b_in, c_in = _inputs(3, 1, 6, 8, seed=1)
    y, _, h = oracle.scan_fwd(x, dt, aneg, b_in, c_in)
    expect = dt[:, 0] * x[:, 0] * (c_in[:, 0] * b_in[:, 0]).sum(-1)[:, None]
    np.testing.assert_allclose(y[:, 0], expect, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(h, (dt * x)[:, 0, :, None] * b_in[:, 0, None, :], rtol=1e-13)


def test_zero_decay_is_a_prefix_sum():
    x, dt, aneg, b_in, c_in = _inputs(2, 25, 4, 6, seed=2)
    aneg = np.zeros_like(aneg)
    y, _, h_last = oracle.scan_fwd(x, dt, aneg, b_in, c_in)
    h = np.cumsum((dt * x)[..., None] * b_in[:, :, None, :], axis=1)
    np.testing.assert_allclose(y, (h * c_in[:, :, None, :]).sum(-1), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(h_last, h[:, -1], rtol=1e-12, atol=1e-12)


def test_constant_inputs_give_a_geometric_series():
    bt, t_len, d, n = 1, 30, 2, 3
    x = np.full((bt, t_len, d), 0.7)
    dt = np.full((bt, t_len, d), 0.05)
    aneg = np.array([[1.0, 2.0, 3.0], [0.5, 4.0, 8.0]])
    b_in = np.tile(np.array([0.3, -1.2, 2.0]), (bt, t_len, 1))
    c_in = np.ones((bt, t_len, n))
    _, _, h_last = oracle.scan_fwd(x, dt, aneg, b_in, c_in)
    a = np.exp(-0.05 * aneg)                       # (d, n)
    b = 0.05 * 0.7 * np.array([0.3, -1.2, 2.0])    # (n,)
    expect = b * (1 - a ** t_len) / (1 - a)
    np.testing.assert_allclose(h_last[0], expect, rtol=1e-12)


def test_zero_input_gives_zero_output():
    x, dt, aneg, b_in, c_in = _inputs(2, 19, 5, 4, seed=3)
    y, _, h = oracle.scan_fwd(np.zeros_like(x), dt, aneg, b_in, c_in)
    assert not y.any() and not h.any()


def test_forward_is_linear_in_x():
    x, dt, aneg, b_in, c_in = _inputs(2, 21, 5, 4, seed=4)
    x2 = _inputs(2, 21, 5, 4, seed=5)[0]
    y1 = oracle.scan_fwd(x, dt, aneg, b_in, c_in)[0]
    y2 = oracle.scan_fwd(x2, dt, aneg, b_in, c_in)[0]
    y12 = oracle.scan_fwd(2.5 * x - 0.5 * x2, dt, aneg, b_in, c_in)[0]
    np.testing.assert_allclose(y12, 2.5 * y1 - 0.5 * y2, rtol=1e-11, atol=1e-12)


def test_forward_is_causal():
    arrs = _inputs(1, 30, 4, 4, seed=6)
    y = oracle.scan_fwd(*arrs)[0]
    pert = [a.copy() for a in arrs]
    for i in (0, 1, 3, 4):
        pert[i][:, 12:] += 1.0
    y2 = oracle.scan_fwd(*pert)[0]
    assert np.array_equal(y[:, :12], y2[:, :12])
    assert not np.allclose(y[:, 12:], y2[:, 12:])


@pytest.mark.parametrize("chunk", [1, 4, 7, 16, 30, 64])
def test_checkpoints_are_the_state_at_each_chunk_end(chunk):
    arrs = _inputs(2, 30, 3, 4, seed=7)
    _, ckpt, h_last = oracle.scan_fwd(*arrs, chunk=chunk)
    h = _h_all(*arrs)
    ends = [min((c + 1) * chunk, 30) - 1 for c in range((30 + chunk - 1) // chunk)]
    assert ckpt.shape == (2, len(ends), 3, 4)
    np.testing.assert_allclose(ckpt, h[:, ends], rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(h_last, h[:, -1], rtol=1e-13, atol=1e-15)


def test_decode_steps_chain_to_the_scan():
    arrs = _inputs(2, 23, 5, 8, seed=8)
    y, _, _ = oracle.scan_fwd(*arrs)
    h = _h_all(*arrs)
    np.testing.assert_allclose(y, (h * arrs[4][:, :, None, :]).sum(-1), rtol=1e-12, atol=1e-14)


def test_state_passing_continues_the_scan():
    """Scanning [:t0], then stepping on from its h_last, equals the full scan."""
    x, dt, aneg, b_in, c_in = _inputs(1, 26, 4, 4, seed=9)
    y_full = oracle.scan_fwd(x, dt, aneg, b_in, c_in)[0]
    _, _, h = oracle.scan_fwd(x[:, :11], dt[:, :11], aneg, b_in[:, :11], c_in[:, :11])
    for t in range(11, 26):
        h, yt = oracle.scan_step(h, x[:, t], dt[:, t], aneg, b_in[:, t], c_in[:, t])
        np.testing.assert_allclose(yt, y_full[:, t], rtol=1e-12, atol=1e-14)


# ----------------------------------------------------------------- backward

def _loss(arrs, dy, dh=None):
    y, _, h_last = oracle.scan_fwd(*arrs)
    v = float((y * dy).sum())
    if dh is not None:
        v += float((h_last * dh).sum())
    return v


def _fd_check(grads, arrs, dy, dh=None, per_tensor=8, seed=0, eps=1e-6):
    """max relative deviation of grads from central differences."""
    rng = np.random.default_rng(seed)
    worst = 0.0
    for i, (g, a) in enumerate(zip(grads, arrs)):
        flat = a.reshape(-1)
        for j in rng.permutation(flat.size)[:per_tensor]:
            p, m = [t.copy() for t in arrs], [t.copy() for t in arrs]
            p[i].reshape(-1)[j] += eps
            m[i].reshape(-1)[j] -= eps
            fd = (_loss(p, dy, dh) - _loss(m, dy, dh)) / (2 * eps)
            scale = max(np.abs(g).max(), 1e-12)
            worst = max(worst, abs(g.reshape(-1)[j] - fd) / scale)
    return worst


@pytest.mark.parametrize("shape", [(1, 9, 3, 4), (2, 14, 2, 5)])
def test_gradients_match_finite_differences(shape):
    arrs = _inputs(*shape, seed=11)
    dy = np.random.default_rng(12).standard_normal(arrs[0].shape)
    grads = oracle.scan_bwd(*arrs, dy)
    assert _fd_check(grads, arrs, dy) < 1e-7


def test_state_gradient_matches_finite_differences():
    arrs = _inputs(1, 12, 3, 4, seed=13)
    rng = np.random.default_rng(14)
    dy = rng.standard_normal(arrs[0].shape)
    dh = rng.standard_normal((1, 3, 4))
    grads = oracle.scan_bwd(*arrs, dy, dh_last=dh)
    assert _fd_check(grads, arrs, dy, dh) < 1e-7


def test_vjp_dot_product():
    """<dy, J v> == <J^T dy, v> for a random direction v over all inputs."""
    arrs = _inputs(2, 16, 3, 4, seed=15)
    rng = np.random.default_rng(16)
    dy = rng.standard_normal(arrs[0].shape)
    v = [rng.standard_normal(a.shape) for a in arrs]
    eps = 1e-6
    yp = oracle.scan_fwd(*[a + eps * w for a, w in zip(arrs, v)])[0]
    ym = oracle.scan_fwd(*[a - eps * w for a, w in zip(arrs, v)])[0]
    jv = ((yp - ym) / (2 * eps) * dy).sum()
    vjp = sum(float((g * w).sum()) for g, w in zip(oracle.scan_bwd(*arrs, dy), v))
    assert abs(jv - vjp) <= 1e-7 * max(1.0, abs(vjp))


def test_dc_is_dy_times_state_summed_over_channels():
    arrs = _inputs(2, 13, 4, 3, seed=17)
    dy = np.random.default_rng(18).standard_normal(arrs[0].shape)
    dc = oracle.scan_bwd(*arrs, dy)[4]
    h = _h_all(*arrs)
    np.testing.assert_allclose(dc, np.einsum("btd,btdn->btn", dy, h), rtol=1e-12, atol=1e-14)


# ------------------------------------------------------- planted mistakes

def test_checks_reject_planted_mistakes():
    """Each pin above fails for a plausible slip in the oracle."""
    arrs = _inputs(1, 10, 3, 4, seed=19)
    dy = np.random.default_rng(20).standard_normal(arrs[0].shape)
    grads = list(oracle.scan_bwd(*arrs, dy))
    # Transposed operands: B and C swapped in the forward.
    x, dt, aneg, b_in, c_in = arrs
    y_swapped = oracle.scan_fwd(x, dt, aneg, c_in, b_in)[0]
    y_cf = oracle.scan_fwd_closed_form(*arrs)[0]
    assert np.abs(y_swapped - y_cf).max() > 1e-3
    # Wrong sign of the decay (exp(+dt*Aneg)).
    assert np.abs(oracle.scan_fwd(x, dt, -aneg, b_in, c_in)[0] - y_cf).max() > 1e-3
    # Gradient mistakes: dB and dC exchanged, dAneg sign flipped, ddt missing
    # its x * sum(G*B) term (ddt - dx * x / dt).
    bad_bc = grads[:3] + [grads[4], grads[3]]
    assert _fd_check(bad_bc, arrs, dy) > 1e-2
    bad_sign = grads[:2] + [-grads[2]] + grads[3:]
    assert _fd_check(bad_sign, arrs, dy) > 1e-2
    bad_ddt = [grads[0], grads[1] - grads[0] * x / dt] + grads[2:]
    assert _fd_check(bad_ddt, arrs, dy) > 1e-2
    # The dC pin rejects dC computed from the pre-update state.
    h = _h_all(*arrs)
    h_prev = np.concatenate([np.zeros_like(h[:, :1]), h[:, :-1]], axis=1)
    assert np.abs(np.einsum("btd,btdn->btn", dy, h_prev) - grads[4]).max() > 1e-3


# ------------------------------------------------ conv1d + SiLU (oracle_conv_*)

def _silu(v):
    return v / (1.0 + np.exp(-v))


def _conv_inputs(bt, t_len, d, k, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((bt, t_len, d)), 0.5 * rng.standard_normal((d, k)),
            0.1 * rng.standard_normal(d))


@pytest.mark.parametrize("shape", [(2, 9, 3, 4), (1, 2, 5, 4), (1, 17, 2, 1), (2, 12, 3, 7)])
def test_conv_matches_numpy_convolve(shape):
    """pre[t] = bias + sum_k w[k] x[t-K+1+k] is numpy's full convolution with the
    reversed kernel, cut to the first T outputs (the causal Conv1d)."""
    x, w, bias = _conv_inputs(*shape, seed=31)
    out = oracle.conv_fwd(x, w, bias)
    bt, t_len, d, k = shape
    ref = np.empty_like(out)
    for b in range(bt):
        for c in range(d):
            ref[b, :, c] = _silu(np.convolve(x[b, :, c], w[c, ::-1])[:t_len] + bias[c])
    np.testing.assert_allclose(out, ref, rtol=1e-13, atol=1e-15)
    # A planted mistake: the kernel not reversed (an anti-causal filter) fails.
    bad = _silu(np.convolve(x[0, :, 0], w[0])[:t_len] + bias[0])
    if k > 1:
        assert np.abs(bad - out[0, :, 0]).max() > 1e-3


def test_conv_kernel_one_is_pointwise():
    x, w, bias = _conv_inputs(2, 6, 4, 1, seed=32)
    np.testing.assert_allclose(oracle.conv_fwd(x, w, bias), _silu(bias + w[:, 0] * x), rtol=1e-13)


def test_conv_is_causal():
    x, w, bias = _conv_inputs(1, 20, 3, 4, seed=33)
    out = oracle.conv_fwd(x, w, bias)
    x2 = x.copy()
    x2[:, 9:] += 1.0
    out2 = oracle.conv_fwd(x2, w, bias)
    assert np.array_equal(out[:, :9], out2[:, :9]) and not np.allclose(out[:, 9:], out2[:, 9:])


def _conv_fd(grads, arrs, dout, eps=1e-6, per=8, seed=0):
    rng = np.random.default_rng(seed)
    worst = 0.0
    for i, (g, a) in enumerate(zip(grads, arrs)):
        flat = a.reshape(-1)
        for j in rng.permutation(flat.size)[:per]:
            p, m = [t.copy() for t in arrs], [t.copy() for t in arrs]
            p[i].reshape(-1)[j] += eps
            m[i].reshape(-1)[j] -= eps
            fd = ((oracle.conv_fwd(*p) - oracle.conv_fwd(*m)) * dout).sum() / (2 * eps)
            worst = max(worst, abs(g.reshape(-1)[j] - fd) / max(np.abs(g).max(), 1e-12))
    return worst


@pytest.mark.parametrize("shape", [(2, 10, 3, 4), (1, 3, 2, 5)])
def test_conv_gradients_match_finite_differences(shape):
    arrs = list(_conv_inputs(*shape, seed=34))
    dout = np.random.default_rng(35).standard_normal(arrs[0].shape)
    grads = oracle.conv_bwd(*arrs, dout)
    assert _conv_fd(grads, arrs, dout) < 1e-7
    # Planted mistake: the SiLU derivative without its p * (1 - sig(p)) term.
    x, w, bias = arrs
    bt, t_len, d, k = shape
    pre = np.empty_like(x)
    for b in range(bt):
        for c in range(d):
            pre[b, :, c] = np.convolve(x[b, :, c], w[c, ::-1])[:t_len] + bias[c]
    s_bad = dout / (1.0 + np.exp(-pre))
    xp = np.concatenate([np.zeros((bt, k - 1, d)), x], axis=1)       # x[t - K + 1 + k]
    dw_bad = np.stack([(s_bad * xp[:, j:j + t_len]).sum((0, 1)) for j in range(k)], axis=1)
    bad = [grads[0], dw_bad, s_bad.sum((0, 1))]
    assert _conv_fd(bad, arrs, dout) > 1e-2


def test_conv_vjp_dot_product():
    arrs = list(_conv_inputs(2, 11, 3, 4, seed=36))
    rng = np.random.default_rng(37)
    dout = rng.standard_normal(arrs[0].shape)
    v = [rng.standard_normal(a.shape) for a in arrs]
    eps = 1e-6
    jv = ((oracle.conv_fwd(*[a + eps * u for a, u in zip(arrs, v)])
           - oracle.conv_fwd(*[a - eps * u for a, u in zip(arrs, v)])) / (2 * eps) * dout).sum()
    vjp = sum(float((g * u).sum()) for g, u in zip(oracle.conv_bwd(*arrs, dout), v))
    assert abs(jv - vjp) <= 1e-7 * max(1.0, abs(vjp))


# ------------------------------- dt gate + softplus(A) (oracle.scan_gated_*)

LO, HI = 0.001, 0.1   # the reference's MambaConfig dt_min, dt_max (model.py:53-54)


def _gated_inputs(bt, t_len, d, n, seed):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal((bt, t_len, d)), rng.standard_normal((bt, t_len, d)),
            np.tile(np.arange(1.0, n + 1), (d, 1)) + 0.3 * rng.standard_normal((d, n)),
            rng.standard_normal((bt, t_len, n)), rng.standard_normal((bt, t_len, n))]


def _gated_fd(grads, arrs, dy, eps=1e-6, per=8, seed=0):
    rng = np.random.default_rng(seed)
    worst = 0.0
    for i, (g, a) in enumerate(zip(grads, arrs)):
        flat = a.reshape(-1)
        for j in rng.permutation(flat.size)[:per]:
            p, m = [t.copy() for t in arrs], [t.copy() for t in arrs]
            p[i].reshape(-1)[j] += eps
            m[i].reshape(-1)[j] -= eps
            fd = ((oracle.scan_gated_fwd(*p, LO, HI)[0] - oracle.scan_gated_fwd(*m, LO, HI)[0])
                  * dy).sum() / (2 * eps)
            worst = max(worst, abs(g.reshape(-1)[j] - fd) / max(np.abs(g).max(), 1e-12))
    return worst


def test_gate_and_softplus_closed_forms():
    np.testing.assert_allclose(oracle.gate_dt(np.array([0.0]), LO, HI), [(LO + HI) / 2], rtol=1e-15)
    np.testing.assert_allclose(oracle.gate_dt(np.array([-800.0, 800.0]), LO, HI), [LO, HI],
                               rtol=1e-15)
    np.testing.assert_allclose(oracle.softplus(np.array([0.0])), [np.log(2.0)], rtol=1e-15)
    # Large a: softplus(a) = a + log1p(e^-a); very negative a: e^a (no underflow to 0).
    np.testing.assert_allclose(oracle.softplus(np.array([40.0, -40.0])),
                               [40.0 + np.exp(-40.0), np.exp(-40.0)], rtol=1e-12)


@pytest.mark.parametrize("shape", [(1, 9, 3, 4), (2, 14, 2, 5)])
def test_gated_gradients_match_finite_differences(shape):
    arrs = _gated_inputs(*shape, seed=41)
    dy = np.random.default_rng(42).standard_normal(arrs[0].shape)
    grads = list(oracle.scan_gated_bwd(*arrs, LO, HI, dy))
    assert _gated_fd(grads, arrs, dy) < 1e-6
    # Planted mistakes: the gate's span factor dropped; sigmoid'(raw) taken as
    # sigmoid(raw); softplus' taken as 1 (dA = dAneg).
    raw = arrs[1]
    s = 1.0 / (1.0 + np.exp(-raw))
    assert _gated_fd([grads[0], grads[1] / (HI - LO)] + grads[2:], arrs, dy) > 1e-2
    assert _gated_fd([grads[0], grads[1] / (1.0 - s)] + grads[2:], arrs, dy) > 1e-2
    daneg = oracle.scan_bwd(arrs[0], oracle.gate_dt(raw, LO, HI), oracle.softplus(arrs[2]),
                            arrs[3], arrs[4], dy)[2]
    assert _gated_fd(grads[:2] + [daneg] + grads[3:], arrs, dy) > 1e-2


def test_gated_gradients_match_torch_autograd():
    """The chain rule through the gate and softplus against torch's float64
    autograd of the same expressions (dt and Aneg enter the scan as leaves)."""
    import torch
    arrs = _gated_inputs(2, 11, 3, 4, seed=43)
    dy = np.random.default_rng(44).standard_normal(arrs[0].shape)
    raw = torch.tensor(arrs[1], requires_grad=True)
    a = torch.tensor(arrs[2], requires_grad=True)
    dt = LO + (HI - LO) * torch.sigmoid(raw)
    aneg = torch.nn.functional.softplus(a)
    _, ddt, daneg, _, _ = oracle.scan_bwd(arrs[0], dt.detach().numpy(), aneg.detach().numpy(),
                                          arrs[3], arrs[4], dy)
    torch.autograd.backward([dt, aneg], [torch.tensor(ddt), torch.tensor(daneg)])
    got = oracle.scan_gated_bwd(*arrs, LO, HI, dy)
    np.testing.assert_allclose(got[1], raw.grad.numpy(), rtol=1e-12, atol=1e-300)
    np.testing.assert_allclose(got[2], a.grad.numpy(), rtol=1e-12, atol=1e-300)


# ---------------------------------- output gate (oracle.out_gate_*)

def test_out_gate_closed_forms():
    rng = np.random.default_rng(45)
    y, d = rng.standard_normal((2, 5, 3)), rng.standard_normal(3)
    assert np.all(oracle.out_gate_fwd(y, d, np.zeros_like(y)) == 0.0)
    # silu(z) -> z for large z: out = (y + D) * z
    z = np.full_like(y, 60.0)
    np.testing.assert_allclose(oracle.out_gate_fwd(y, d, z), (y + d) * 60.0, rtol=1e-14)
    # silu(1) = 1 / (1 + e^-1)
    np.testing.assert_allclose(oracle.out_gate_fwd(np.ones((1, 1, 1)), np.zeros(1),
                                                   np.ones((1, 1, 1))), [[[1 / (1 + np.exp(-1))]]])


def test_out_gate_gradients_match_finite_differences():
    rng = np.random.default_rng(46)
    arrs = [rng.standard_normal((2, 7, 3)), rng.standard_normal(3), rng.standard_normal((2, 7, 3))]
    dout = rng.standard_normal((2, 7, 3))
    dy, dd, dz = oracle.out_gate_bwd(*arrs, dout)

    def fd_check(grads):
        worst, eps = 0.0, 1e-6
        for i, g in enumerate(grads):
            for j in range(arrs[i].size):
                p, m = [t.copy() for t in arrs], [t.copy() for t in arrs]
                p[i].reshape(-1)[j] += eps
                m[i].reshape(-1)[j] -= eps
                fd = ((oracle.out_gate_fwd(*p) - oracle.out_gate_fwd(*m)) * dout).sum() / (2 * eps)
                worst = max(worst, abs(g.reshape(-1)[j] - fd) / max(np.abs(g).max(), 1e-12))
        return worst

    assert fd_check([dy, dd, dz]) < 1e-7
    # Planted mistakes: silu' without its z * (1 - s) term; dD_skip not summed
    # over time (last step only).
    y, dsk, z = arrs
    s = 1.0 / (1.0 + np.exp(-z))
    assert fd_check([dy, dd, dout * (y + dsk) * s]) > 1e-2
    assert fd_check([dy, dy[:, -1].sum(0), dz]) > 1e-2
