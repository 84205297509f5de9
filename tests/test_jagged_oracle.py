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
