"""The backward oracle pinned the way the reference pins its own backward kernels: autograd through
the forward (recir/ops/helion/jagged_hstu_attention.py:260-280).

Three independent checks of oracle/hstu_oracle.c:hstu_oracle_attn_bwd, none of which retypes its
formulas: (1) golden gradients from torch autograd through the reference's compiled C++ forward
operator, (2) torch autograd through a dense float64 restatement of the forward (covers the score
bias and the prefix contextual rule, which the reference operator does not have), (3) central finite
differences of the forward oracle.  A wrong sign, a dropped silu' term, a missing alpha or scale, or
a transposed dK/dQ fails all three.
"""
import os

import numpy as np
import pytest
import torch

from tests.golden.cases import SMALL_CASES, build_inputs, fixture_file, upstream_gradient

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _scale_arg(scale):
    if scale is None:
        return None
    return scale.numpy() if scale.dim() else np.float32(scale.item())


def _oracle_bwd(oracle, case, ctx_mode=None, **kw):
    wl, scale, nt = build_inputs(case)
    dout = upstream_gradient(case, wl)
    mode = oracle.CTX_REFCPP if ctx_mode is None else ctx_mode
    grads = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                            None if nt is None else nt.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                            attn_scale=_scale_arg(scale), contextual_seq_len=case["ctx"], ctx_mode=mode,
                            max_attn_len=case["max_attn_len"], full_attn_size=case["full_attn_size"],
                            mask_type=case["mask_type"], **kw)
    return wl, dout, grads


@pytest.mark.parametrize("name", sorted(n for n, c in SMALL_CASES.items() if c["Dqk"] < 128))
def test_backward_oracle_matches_reference_autograd_golden(oracle, name):
    fx = np.load(os.path.join(GOLDEN, fixture_file(SMALL_CASES[name], backward=True)))
    wl, _dout, grads = _oracle_bwd(oracle, SMALL_CASES[name])
    end = int(wl.seq_offsets[-1])
    for g, key in zip(grads, ("dq", "dk", "dv")):
        want = fx[f"{name}/{key}"]
        scale = max(1.0, float(np.abs(want).max()))
        np.testing.assert_allclose(g, want, rtol=2e-5, atol=2e-6 * scale, err_msg=key)
        assert not g[end:].any()  # tail rows get no gradient


@pytest.mark.parametrize("name", ["per_token_scale", "d128_mixed", "d128_ctx_refrule", "d128_semilocal",
                                  "sl_window_and_tail", "nc_d128", "nc_window_and_tail"])
def test_live_reference_autograd_when_built(oracle, name):
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built")
    case = SMALL_CASES[name]
    wl, scale, nt = build_inputs(case)
    dout = upstream_gradient(case, wl)
    q, k, v = (t.clone().requires_grad_(True) for t in (wl.q, wl.k, wl.v))
    out = oracle.ref_attn_fwd(q, k, v, wl.seq_offsets, nt, max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                              attn_scale=scale, contextual_seq_len=case["ctx"],
                              max_attn_len=case["max_attn_len"], full_attn_size=case["full_attn_size"],
                              mask_type=case["mask_type"])
    out.backward(dout[: out.shape[0]])
    _, _, grads = _oracle_bwd(oracle, case)
    for g, want in zip(grads, (q.grad, k.grad, v.grad)):
        np.testing.assert_allclose(g, want.numpy(), rtol=5e-5, atol=2e-6 * max(1.0, float(want.abs().max())))


def _dense_forward_f64(q, k, v, lengths, targets, N, alpha, scale, rab, ctx):
    """Dense float64 torch forward, one sequence at a time, prefix contextual rule, optional bias."""
    outs = []
    s = 0
    for n, t in zip(lengths, targets):
        qs, ks, vs = q[s:s + n], k[s:s + n], v[s:s + n]
        m = torch.arange(n).view(n, 1)
        j = torch.arange(n).view(1, n)
        keep = (m == j) | ((m >= j) & (j < n - t)) | (j < ctx)
        S = alpha * torch.einsum("mhd,jhd->hmj", qs, ks)
        if rab is not None:
            S = S + rab[:, (m - j + N - 1)]
        P = torch.nn.functional.silu(S) * scale * keep
        outs.append(torch.einsum("hmj,jhd->mhd", P, vs))
        s += n
    return torch.cat(outs) if outs else q.new_zeros((0,) + v.shape[1:])


@pytest.mark.parametrize("ctx,with_rab", [(0, False), (3, False), (0, True), (5, True)])
def test_backward_oracle_matches_dense_torch_autograd(oracle, ctx, with_rab):
    rng = np.random.default_rng(5 + ctx)
    lengths, targets, N, H, Dqk, Dv, alpha, scale = [7, 1, 0, 12, 5], [2, 0, 0, 4, 5], 12, 3, 8, 6, 0.23, 0.11
    T = sum(lengths) + 2  # two tail rows
    off = np.concatenate([[0], np.cumsum(lengths)])
    q, k = (rng.standard_normal((T, H, Dqk)) for _ in range(2))
    v, g = (rng.standard_normal((T, H, Dv)) for _ in range(2))
    rab = rng.standard_normal((H, 2 * N - 1)) if with_rab else None
    tq, tk, tv = (torch.tensor(x.astype(np.float32).astype(np.float64), requires_grad=True) for x in (q, k, v))
    trab = None if rab is None else torch.tensor(rab.astype(np.float32).astype(np.float64), requires_grad=True)
    out = _dense_forward_f64(tq, tk, tv, lengths, targets, N, alpha, scale, trab, ctx)
    out.backward(torch.tensor(g.astype(np.float32).astype(np.float64))[: out.shape[0]])
    res = oracle.attn_bwd(g, q, k, v, off, targets, max_seq_len=N, alpha=alpha, attn_scale=np.float32(scale),
                          rab=rab, contextual_seq_len=ctx, ctx_mode=oracle.CTX_PREFIX, rab_grad=with_rab)
    # attn_scale travels as float32
    for got, want in zip(res[:3], (tq.grad, tk.grad, tv.grad)):
        np.testing.assert_allclose(got, want.numpy(), rtol=1e-5, atol=1e-6)
        assert not got[off[-1]:].any()
    if with_rab:
        # gradient of the bias table: autograd through the dense form's gather rab[:, m - j + N - 1]
        want = trab.grad.numpy()
        assert np.abs(want).max() > 0.1  # the table matters in this case
        np.testing.assert_allclose(res[3], want, rtol=1e-5, atol=1e-6)
        longest = max(lengths)
        assert not res[3][:, : N - longest].any() and not res[3][:, N + longest - 1:].any()  # diagonals no pair has


def test_backward_oracle_matches_finite_differences_of_forward_oracle(oracle):
    rng = np.random.default_rng(11)
    lengths, targets, N, H, Dqk, Dv, alpha = [6, 4, 1], [2, 4, 0], 8, 2, 4, 3, 0.4
    off = np.concatenate([[0], np.cumsum(lengths)])
    T = int(off[-1])
    q, k = (rng.standard_normal((T, H, Dqk)).astype(np.float32) for _ in range(2))
    v, g = (rng.standard_normal((T, H, Dv)).astype(np.float32) for _ in range(2))
    rab = rng.standard_normal((H, 2 * N - 1)).astype(np.float32)
    kw = dict(max_seq_len=N, alpha=alpha, attn_scale=np.float32(0.3), rab=rab, contextual_seq_len=2,
              ctx_mode=oracle.CTX_PREFIX)

    def loss(q_, k_, v_):
        return float((oracle.attn_fwd(q_, k_, v_, off, targets, **kw).astype(np.float64) * g).sum())

    grads = oracle.attn_bwd(g, q, k, v, off, targets, **kw)
    eps = 1e-2
    for which, (x, grad) in enumerate(zip((q, k, v), grads)):
        idx = [tuple(rng.integers(0, s) for s in x.shape) for _ in range(24)]
        for i in idx:
            xp, xm = x.copy(), x.copy()
            xp[i] += eps
            xm[i] -= eps
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[which], args_m[which] = xp, xm
            fd = (loss(*args_p) - loss(*args_m)) / (float(xp[i]) - float(xm[i]))
            assert abs(fd - grad[i]) <= 2e-3 * max(1.0, abs(fd)), (which, i, fd, grad[i])


def test_backward_linear_in_upstream_gradient_and_zero_for_masked_keys(oracle):
    case = SMALL_CASES["all_targets"]  # every key is a target: only the diagonal is kept
    wl, dout, (dq, dk, dv) = _oracle_bwd(oracle, case)
    wl2, scale, nt = build_inputs(case)
    g2 = oracle.attn_bwd(2.0 * dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                         nt.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha, attn_scale=_scale_arg(scale))
    for a, b in zip((dq, dk, dv), g2):
        np.testing.assert_allclose(2.0 * a, b, rtol=1e-6, atol=1e-7)
    # diagonal only: dv[j] = p(j,j) * dout[j], a per-token closed form
    qn, kn = wl.q.numpy().astype(np.float64), wl.k.numpy().astype(np.float64)
    x = wl.alpha * (qn * kn).sum(-1)
    p = x / (1.0 + np.exp(-x)) * float(scale)
    np.testing.assert_allclose(dv, p[..., None] * dout.numpy(), rtol=1e-5, atol=1e-6)
