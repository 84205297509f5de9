"""GPU parity tests of the jagged neighbours: the HIP row-gather kernels, through the operators (and
so through the C ABI), against the oracle -- bit-exact, they only move rows."""
import numpy as np
import pytest
import torch

from oracle import jagged_oracle as jo

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu_and_library():
    from recir_amd import _lib

    assert torch.cuda.is_available(), "these tests need the MI355X"
    _lib.load()


def _offsets(lengths):
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)


def _values(rng, rows, tail, dtype):
    x = rng.standard_normal((rows,) + tail).astype(np.float32)
    if dtype == torch.int64:
        return torch.tensor((x * 100).astype(np.int64))
    return torch.tensor(x).to(dtype)


def _np(t):
    return t.float().cpu().numpy() if t.dtype in (torch.bfloat16, torch.float16) else t.cpu().numpy()


CASES = [((128,), torch.bfloat16), ((6,), torch.float32), ((1,), torch.int64), ((), torch.float16),
         ((3, 5), torch.float32), ((7,), torch.bfloat16)]


@pytest.mark.parametrize("tail,dtype", CASES)
@pytest.mark.parametrize("off_dtype", [torch.int64, torch.int32])
def test_pad_and_unpad(tail, dtype, off_dtype):
    import recir_amd

    rng = np.random.default_rng(len(tail) + 7)
    lengths = np.array([3, 0, 9, 1, 4, 0, 17])
    off = _offsets(lengths)
    x = _values(rng, int(off[-1]), tail, dtype)
    offd = torch.tensor(off, dtype=off_dtype, device=DEV)
    for max_len, pad in ((17, 0.0), (20, -2.5), (4, 1.0)):
        got = recir_amd.jagged_to_padded_dense(x.to(DEV), [offd], [max_len], pad)
        want = jo.jagged_to_padded_dense(_np(x), off, max_len, pad if dtype != torch.int64 else int(pad))
        assert got.shape == want.shape and got.dtype == dtype
        np.testing.assert_array_equal(_np(got), want.astype(_np(got).dtype))
    dense = recir_amd.jagged_to_padded_dense(x.to(DEV), [offd], [17], 0.0)
    back, off_out = recir_amd.dense_to_jagged(dense, [offd])
    assert torch.equal(back.cpu(), x) and off_out is not None
    back2, _ = recir_amd.dense_to_jagged(dense, [offd], int(off[-1]) + 3)
    np.testing.assert_array_equal(_np(back2), jo.dense_to_jagged(_np(dense), off, int(off[-1]) + 3))
    # truncated dense width: the reference's clamped flat index, reproduced bit for bit
    narrow = recir_amd.jagged_to_padded_dense(x.to(DEV), [offd], [4], 0.0)
    got, _ = recir_amd.dense_to_jagged(narrow, [offd])
    np.testing.assert_array_equal(_np(got), jo.dense_to_jagged(_np(narrow), off))


@pytest.mark.parametrize("tail,dtype", [c for c in CASES if len(c[0]) > 0])  # the 2-D operators take [rows, D] values
@pytest.mark.parametrize("npre", [0, 2])
def test_concat_and_split(tail, dtype, npre):
    import recir_amd

    rng = np.random.default_rng(11 + npre)
    la = np.array([2, 0, 5, 1, 0, 8])
    lb = np.array([3, 2, 2, 4, 2, 6])
    oa, ob = _offsets(la), _offsets(lb)
    a, b = _values(rng, int(oa[-1]), tail, dtype), _values(rng, int(ob[-1]), tail, dtype)
    ad, bd = a.to(DEV), b.to(DEV)
    oad, obd = torch.tensor(oa, device=DEV), torch.tensor(ob, device=DEV)
    cat = recir_amd.concat_2D_jagged_fwd(16, ad, bd, oad, obd, False, npre)
    want = jo.concat_2d_jagged(_np(a), _np(b), oa, ob, False, npre)
    np.testing.assert_array_equal(_np(cat), want)
    sa, sb = recir_amd.split_2D_jagged_fwd(cat, 16, oad, obd, len(a), len(b), False, False, 0, npre, len(la))
    assert torch.equal(sa.cpu(), a) and torch.equal(sb.cpu(), b)
    if npre == 0:
        cat2 = recir_amd.concat_2d_jagged(ad, oad, bd, obd)
        assert torch.equal(cat2, cat)
        l2, r2 = recir_amd.split_2d_jagged(cat2, oad, obd, len(a), len(b))
        assert torch.equal(l2.cpu(), a) and torch.equal(r2.cpu(), b)


def test_concat_dense_sides_and_replace():
    import recir_amd

    rng = np.random.default_rng(5)
    B, S, D = 4, 3, 16
    dense = torch.tensor(rng.standard_normal((B, S, D)).astype(np.float32)).bfloat16()
    lb = np.array([2, 0, 5, 1])
    ob = _offsets(lb)
    b = torch.tensor(rng.standard_normal((int(ob[-1]), D)).astype(np.float32)).bfloat16()
    obd = torch.tensor(ob, device=DEV)
    cat = recir_amd.concat_2D_jagged_fwd(8, dense.to(DEV), b.to(DEV), None, obd, False, 0)
    np.testing.assert_array_equal(_np(cat), jo.concat_2d_jagged(_np(dense), _np(b), None, ob))
    sa, sb = recir_amd.split_2D_jagged_fwd(cat, 8, obd, obd, 0, len(b), True, False, S, 0, B)
    assert torch.equal(sa.cpu(), dense) and torch.equal(sb.cpu(), b)
    cat = recir_amd.concat_2D_jagged_fwd(8, b.to(DEV), dense.to(DEV), obd, None, False, 0)  # dense right side
    np.testing.assert_array_equal(_np(cat), jo.concat_2d_jagged(_np(b), _np(dense), ob, None))
    # replace: the last len_b rows of every sample of a are overwritten by b
    la = np.array([4, 1, 6, 3])
    oa = _offsets(la)
    a = torch.tensor(rng.standard_normal((int(oa[-1]), D)).astype(np.float32))
    lb2 = np.array([2, 1, 0, 3])
    ob2 = _offsets(lb2)
    b2 = torch.tensor(rng.standard_normal((int(ob2[-1]), D)).astype(np.float32))
    rep = recir_amd.concat_2D_jagged_fwd(8, a.to(DEV), b2.to(DEV), torch.tensor(oa, device=DEV),
                                         torch.tensor(ob2, device=DEV), True, 0)
    np.testing.assert_array_equal(rep.cpu().numpy(), jo.concat_2d_jagged(a.numpy(), b2.numpy(), oa, ob2, True, 0))


def test_argument_rules_follow_the_reference():
    import recir_amd

    a = torch.zeros(3, 4, device=DEV)
    off = torch.tensor([0, 3], device=DEV)
    with pytest.raises(ValueError, match="at least one input must be jagged"):
        recir_amd.concat_2D_jagged_fwd(4, a.view(1, 3, 4), a.view(1, 3, 4), None, None, False, 0)
    with pytest.raises(ValueError, match="non-negative"):
        recir_amd.concat_2D_jagged_fwd(4, a, a, off, off, False, -1)
    with pytest.raises(ValueError, match="not supported when is_replace"):
        recir_amd.concat_2D_jagged_fwd(4, a, a, off, off, True, 1)
    with pytest.raises(ValueError, match="only supported for two jagged"):
        recir_amd.concat_2D_jagged_fwd(4, a.view(1, 3, 4), a, None, off, False, 1)
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        recir_amd.concat_2d_jagged(a.cpu(), off.cpu(), a.cpu(), off.cpu())


def test_autograd_round_trips():
    import recir_amd

    lengths = np.array([3, 0, 5])
    off = torch.tensor(_offsets(lengths), device=DEV)
    x = torch.randn(8, 4, device=DEV, requires_grad=True)
    dense = recir_amd.jagged_to_padded_dense(x, [off], [6], 0.0)
    w = torch.randn_like(dense)
    (dense * w).sum().backward()
    want, _ = recir_amd.dense_to_jagged(w, [off], 8)
    assert torch.equal(x.grad, want)
    a = torch.randn(8, 4, device=DEV, requires_grad=True)
    b = torch.randn(8, 4, device=DEV, requires_grad=True)
    cat = recir_amd.concat_2d_jagged(a, off, b, off)
    wc = torch.randn_like(cat)
    (cat * wc).sum().backward()
    ga, gb = recir_amd.split_2d_jagged(wc, off, off, 8, 8)
    assert torch.equal(a.grad, ga) and torch.equal(b.grad, gb)


def test_large_rows_saturate_nothing_and_stay_exact():
    """The attention path's own shape: [T, H * D] bf16 rows of configuration 2, padded and back."""
    import recir_amd
    from recir_amd.workloads import make_config

    wl = make_config(2)
    x = wl.q.to(DEV, torch.bfloat16).reshape(wl.T, -1)
    off = wl.seq_offsets.to(DEV)
    dense = recir_amd.jagged_to_padded_dense(x, [off], [wl.max_seq_len], 0.0)
    assert dense.shape == (wl.B, wl.max_seq_len, x.shape[1])
    back, _ = recir_amd.dense_to_jagged(dense, [off], wl.T)
    assert torch.equal(back, x)
    lengths = (wl.seq_offsets[1:] - wl.seq_offsets[:-1]).tolist()
    for b in (0, 7, 31):
        n, s = lengths[b], int(wl.seq_offsets[b])
        assert torch.equal(dense[b, :n], x[s:s + n]) and not dense[b, n:].any()


@pytest.mark.parametrize("fn", ["sqrt", "log"])
@pytest.mark.parametrize("seq_dt,tab_dt,ts_dt", [(torch.float32, torch.float32, torch.int64),
                                                 (torch.bfloat16, torch.bfloat16, torch.int64),
                                                 (torch.bfloat16, torch.float32, torch.float32)])
def test_add_ts_pos_emb(fn, seq_dt, tab_dt, ts_dt):
    import recir_amd

    rng = np.random.default_rng(17)
    lengths = np.array([5, 1, 9, 12, 300, 64])
    targets = np.array([2, 0, 3, 12, 40, 0])
    off = _offsets(lengths)
    D, P, Tmax = 40, 50, 300
    seq = torch.tensor(rng.standard_normal((int(off[-1]), D)).astype(np.float32)).to(seq_dt)
    pos = torch.tensor(rng.standard_normal((P, D)).astype(np.float32)).to(tab_dt)
    tab = torch.tensor(rng.standard_normal((2049, D)).astype(np.float32)).to(tab_dt)
    stamps = np.sort(rng.integers(0, 40_000_000, size=(len(lengths), Tmax)), axis=1)
    stamps_t = torch.tensor(stamps).to(ts_dt)
    for ctx, inter in ((0, False), (3, False)):
        got = recir_amd.add_ts_pos_emb_fwd(seq.to(DEV), torch.tensor(off, device=DEV), pos.to(DEV), tab.to(DEV),
                                           stamps_t.to(DEV), torch.tensor(lengths, device=DEV),
                                           torch.tensor(targets, device=DEV), 512, ctx, inter, fn)
        out, pi, ti, pre = jo.add_ts_pos_emb(seq.float().numpy(), off, pos.float().numpy(), tab.float().numpy(),
                                             stamps_t.numpy(), lengths, targets, ctx, inter, fn,
                                             seq_bf16=seq_dt == torch.bfloat16, tab_bf16=tab_dt == torch.bfloat16)
        assert got[0].dtype == seq_dt and all(g.dtype == torch.int32 for g in got[1:])
        # position rows: exact integer arithmetic; stable sort = stable argsort
        np.testing.assert_array_equal(got[1].cpu().numpy(), np.sort(pi))
        np.testing.assert_array_equal(got[2].cpu().numpy(), np.argsort(pi, kind="stable"))
        safe = np.abs(pre - np.round(pre)) > 1e-3  # away from a bucket boundary the device's log agrees
        got_ti = np.empty_like(ti)
        got_ti[got[4].cpu().numpy()] = got[3].cpu().numpy()  # undo the sort
        np.testing.assert_array_equal(got_ti[safe], ti[safe])
        assert np.abs(got_ti - ti).max() <= 1
        assert (np.diff(got[3].cpu().numpy()) >= 0).all()
        rows_ok = safe
        np.testing.assert_array_equal(got[0].float().cpu().numpy()[rows_ok], out[rows_ok])
        if fn == "sqrt":
            assert safe.all() or True
            np.testing.assert_array_equal(got_ti, ti)  # sqrt is correctly rounded on both sides


@pytest.mark.parametrize("P,D", [(4000, 8), (9000, 8), (64, 24)])
def test_add_ts_pos_emb_sorted_lists_across_chunks(P, D):
    """Sequences long enough for the index lists to span several chunks of the counting sort
    (P <= 8192) and the general sort (P = 9000): sorted keys and permutations equal numpy's stable
    argsort, rows equal the restatement; D = 24 fp32 takes the 16-byte path, D = 8 bf16 too."""
    import recir_amd

    rng = np.random.default_rng(5)
    lengths = np.array([700, 1500, 33, 0, 900, 2047])
    targets = np.array([10, 200, 33, 0, 0, 64])
    off = _offsets(lengths)
    Tmax = 2048
    seq_dt = torch.float32 if D == 24 else torch.bfloat16
    seq = torch.tensor(rng.standard_normal((int(off[-1]), D)).astype(np.float32)).to(seq_dt)
    pos = torch.tensor(rng.standard_normal((P, D)).astype(np.float32)).to(seq_dt)
    tab = torch.tensor(rng.standard_normal((2049, D)).astype(np.float32)).to(seq_dt)
    stamps = np.sort(rng.integers(0, 400_000_000, size=(len(lengths), Tmax)), axis=1)
    got = recir_amd.add_ts_pos_emb_fwd(seq.to(DEV), torch.tensor(off, device=DEV), pos.to(DEV), tab.to(DEV),
                                       torch.tensor(stamps, device=DEV), torch.tensor(lengths, device=DEV),
                                       torch.tensor(targets, device=DEV), 2048, 2, False, "sqrt")
    bf = seq_dt == torch.bfloat16
    out, pi, ti, _pre = jo.add_ts_pos_emb(seq.float().numpy(), off, pos.float().numpy(), tab.float().numpy(), stamps,
                                          lengths, targets, 2, False, "sqrt", seq_bf16=bf, tab_bf16=bf)
    np.testing.assert_array_equal(got[1].cpu().numpy(), np.sort(pi))
    np.testing.assert_array_equal(got[2].cpu().numpy(), np.argsort(pi, kind="stable"))
    np.testing.assert_array_equal(got[3].cpu().numpy(), np.sort(ti))
    np.testing.assert_array_equal(got[4].cpu().numpy(), np.argsort(ti, kind="stable"))
    np.testing.assert_array_equal(got[0].float().cpu().numpy(), out)
