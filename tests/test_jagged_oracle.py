"""The jagged-neighbour oracle (oracle/jagged_oracle.py) pinned against the reference: its own
known-answer tests, its compiled C++ operators on random inputs, round trips, and -- for the two
functions the reference only has in Python -- per-sample slicing written independently here."""
import numpy as np
import pytest
import torch

from oracle import hstu_oracle, jagged_oracle as jo


def test_reference_known_answers_concat():
    # recir/ops/tests/KjtSplitPerFeatureTest.cpp:50-63 (right prefix), :65-77 (replace), :79-91 (dense left)
    a = np.array([10, 11, 20]).reshape(3, 1)
    b = np.array([1, 2, 3, 4, 5]).reshape(5, 1)
    out = jo.concat_2d_jagged(a, b, [0, 2, 3], [0, 3, 5], False, 1)
    assert out.ravel().tolist() == [1, 10, 11, 2, 3, 4, 20, 5]
    a = np.array([10, 11, 12, 20, 21]).reshape(5, 1)
    b = np.array([1, 2, 3]).reshape(3, 1)
    assert jo.concat_2d_jagged(a, b, [0, 3, 5], [0, 1, 3], True, 0).ravel().tolist() == [10, 11, 1, 2, 3]
    a = np.array([10, 11, 20, 21]).reshape(2, 2, 1)
    b = np.array([1, 2, 3]).reshape(3, 1)
    assert jo.concat_2d_jagged(a, b, None, [0, 1, 3], False, 0).ravel().tolist() == [10, 11, 1, 20, 21, 2, 3]


def test_reference_known_answer_split():
    # recir/ops/tests/KjtSplitPerFeatureTest.cpp:177-189
    v = np.array([1, 10, 11, 2, 3, 4, 20, 5]).reshape(8, 1)
    a, b = jo.split_2d_jagged(v, [0, 2, 3], [0, 3, 5], n_prefix_to_right=1)
    assert a.ravel().tolist() == [10, 11, 20] and b.ravel().tolist() == [1, 2, 3, 4, 5]


def _random_pair(rng, B, D, min_b=0):
    la = rng.integers(0, 6, size=B)
    lb = rng.integers(min_b, 7, size=B)
    oa, ob = np.concatenate([[0], np.cumsum(la)]), np.concatenate([[0], np.cumsum(lb)])
    a = rng.standard_normal((int(oa[-1]), D)).astype(np.float32)
    b = rng.standard_normal((int(ob[-1]), D)).astype(np.float32)
    return a, b, oa, ob


@pytest.mark.parametrize("seed", range(6))
def test_oracle_matches_compiled_reference_operators(seed):
    if not hstu_oracle.ref_available():
        pytest.skip("oracle/_ref not built")
    hstu_oracle.ref_op()  # loads the library that also registers the concat / split operators
    rng = np.random.default_rng(seed)
    B, D, npre = int(rng.integers(1, 6)), int(rng.integers(1, 5)), int(rng.integers(0, 3))
    a, b, oa, ob = _random_pair(rng, B, D, min_b=npre)
    ta, tb, toa, tob = torch.tensor(a), torch.tensor(b), torch.tensor(oa), torch.tensor(ob)
    cat = torch.ops.generative_recommenders.concat_2D_jagged_fwd_op(16, ta, tb, toa, tob, False, npre)
    np.testing.assert_array_equal(jo.concat_2d_jagged(a, b, oa, ob, False, npre), cat.numpy())
    sa, sb = torch.ops.generative_recommenders.split_2D_jagged_fwd_op(cat, 16, toa, tob, len(a), len(b), False, False,
                                                                      0, npre, B)
    ga, gb = jo.split_2d_jagged(cat.numpy(), oa, ob, n_prefix_to_right=npre)
    np.testing.assert_array_equal(ga, sa.numpy())
    np.testing.assert_array_equal(gb, sb.numpy())
    np.testing.assert_array_equal(ga, a)
    np.testing.assert_array_equal(gb, b)
    # dense left side (fixed rows per sample) and the replace mode (b never longer than a)
    S = 3
    dense = rng.standard_normal((B, S, D)).astype(np.float32)
    cat = torch.ops.generative_recommenders.concat_2D_jagged_fwd_op(16, torch.tensor(dense), tb, None, tob, False, 0)
    np.testing.assert_array_equal(jo.concat_2d_jagged(dense, b, None, ob, False, 0), cat.numpy())
    sa, sb = torch.ops.generative_recommenders.split_2D_jagged_fwd_op(cat, 16, toa, tob, 0, len(b), True, False, S, 0, B)
    ga, gb = jo.split_2d_jagged(cat.numpy(), None, ob, dense_size_a=S, B=B)
    np.testing.assert_array_equal(ga, sa.numpy())
    np.testing.assert_array_equal(gb, sb.numpy())
    lb2 = np.minimum(np.diff(ob), np.diff(oa))
    ob2 = np.concatenate([[0], np.cumsum(lb2)])
    b2 = rng.standard_normal((int(ob2[-1]), D)).astype(np.float32)
    rep = torch.ops.generative_recommenders.concat_2D_jagged_fwd_op(16, ta, torch.tensor(b2), toa, torch.tensor(ob2), True, 0)
    np.testing.assert_array_equal(jo.concat_2d_jagged(a, b2, oa, ob2, True, 0), rep.numpy())


def test_pad_unpad_against_per_sample_slicing_and_round_trip():
    rng = np.random.default_rng(1)
    lengths = np.array([3, 0, 5, 1, 4])
    off = np.concatenate([[0], np.cumsum(lengths)])
    x = rng.standard_normal((int(off[-1]), 2, 3)).astype(np.float32)
    for max_len in (5, 7, 3):
        dense = jo.jagged_to_padded_dense(x, off, max_len, padding_value=-1.5)
        assert dense.shape == (5, max_len, 2, 3)
        for b, n in enumerate(lengths):
            keep = min(n, max_len)
            np.testing.assert_array_equal(dense[b, :keep], x[off[b]:off[b] + keep])
            assert (dense[b, keep:] == -1.5).all()
    dense = jo.jagged_to_padded_dense(x, off, 6)
    np.testing.assert_array_equal(jo.dense_to_jagged(dense, off), x)  # round trip when nothing is truncated
    # extra rows beyond the last sequence come back as zeros
    back = jo.dense_to_jagged(dense, off, total_L=int(off[-1]) + 2)
    np.testing.assert_array_equal(back[: off[-1]], x)
    assert not back[off[-1]:].any()
    # one-dimensional values
    v = rng.standard_normal(int(off[-1])).astype(np.float32)
    np.testing.assert_array_equal(jo.dense_to_jagged(jo.jagged_to_padded_dense(v, off, 5), off), v)


def test_reference_known_answer_add_ts_pos_emb():
    # recir/ops/tests/KjtSplitPerFeatureTest.cpp:141-175
    seq = np.zeros((3, 1), dtype=np.float32)
    pos = np.array([0.0, 10.0, 20.0, 30.0, 40.0], dtype=np.float32).reshape(5, 1)
    ts_tab = (np.arange(2049, dtype=np.float32) * 100.0).reshape(2049, 1)
    stamps = np.array([[10.0, 40.0, 70.0]], dtype=np.float32)
    out, pi, ti, _ = jo.add_ts_pos_emb(seq, [0, 3], pos, ts_tab, stamps, [3], None, 1, False, "sqrt")
    assert out.ravel().tolist() == [100.0, 30.0, 20.0]
    assert sorted(pi.tolist()) == [0, 2, 3] and sorted(ti.tolist()) == [0, 0, 1]


@pytest.mark.parametrize("fn", ["sqrt", "log"])
@pytest.mark.parametrize("bf16", [False, True])
def test_add_ts_pos_emb_matches_compiled_reference(fn, bf16):
    if not hstu_oracle.ref_available():
        pytest.skip("oracle/_ref not built")
    hstu_oracle.ref_op()
    rng = np.random.default_rng(3)
    lengths = np.array([5, 1, 9, 12])
    targets = np.array([2, 0, 3, 12])
    off = np.concatenate([[0], np.cumsum(lengths)])
    D, P, Tmax = 6, 9, 12
    dt = torch.bfloat16 if bf16 else torch.float32
    seq = torch.tensor(rng.standard_normal((int(off[-1]), D)).astype(np.float32)).to(dt)
    pos = torch.tensor(rng.standard_normal((P, D)).astype(np.float32)).to(dt)
    tab = torch.tensor(rng.standard_normal((2049, D)).astype(np.float32)).to(dt)
    stamps = torch.tensor(np.sort(rng.integers(0, 3_000_000, size=(4, Tmax)), axis=1))
    for ctx, inter in ((0, False), (2, False), (1, True)):
        want = torch.ops.hammer.add_ts_pos_emb_fwd_op(seq, torch.tensor(off), pos, tab, stamps, torch.tensor(lengths),
                                                      torch.tensor(targets // (2 if inter else 1)), 16, ctx, inter, fn)
        out, pi, ti, pre = jo.add_ts_pos_emb(seq.float().numpy(), off, pos.float().numpy(), tab.float().numpy(),
                                             stamps.numpy(), lengths, targets // (2 if inter else 1), ctx, inter, fn,
                                             seq_bf16=bf16, tab_bf16=bf16)
        safe = np.abs(pre - np.round(pre)) > 1e-4  # a logarithm within an ulp of an integer may fall either way
        assert safe.all() or fn == "log"
        np.testing.assert_array_equal(np.sort(pi), want[1].numpy())
        np.testing.assert_array_equal(pi[want[2].numpy()], want[1].numpy())  # the permutation sorts the rows
        if safe.all():
            np.testing.assert_array_equal(np.sort(ti), want[3].numpy())
            np.testing.assert_array_equal(ti[want[4].numpy()], want[3].numpy())
            np.testing.assert_array_equal(out, want[0].float().numpy())
