"""Integer part of the path: the keep mask and the unmasked-pair count (bit-exact by nature).

Pins: two independently written closed forms of the reference mask must agree for every
(n, t, ctx, m, j) with n <= 40 (helion/jagged_hstu_attention.py:192-208 vs the clamp-id form of
kjt_split_per_feature.cpp:639-674 and pallas/hstu_attention.py:86-112); row counts follow the
hand-derived rule "history rows keep m+1 keys, target rows keep cap+1"; the pair count follows the
closed form the FLOP model uses.
"""
import numpy as np
import pytest


def test_two_mask_forms_agree_exhaustively(oracle):
    L = oracle.lib()
    for n in range(0, 41):
        for t in list(range(0, n + 1)) + [n + 1, n + 5]:
            for ctx, mode in ((0, 0), (1, 0), (3, 0), (1, 1), (8, 1)):
                for m in range(n):
                    for j in range(n):
                        a = L.hstu_oracle_keep(m, j, n, t, ctx, mode)
                        b = L.hstu_oracle_keep_clamp_id(m, j, n, t, ctx, mode)
                        assert a == b, (n, t, ctx, mode, m, j)


def test_row_counts_without_prefix(oracle):
    for n in (1, 2, 7, 33):
        for t in (0, 1, n // 2, n):
            cap = n - t
            for m in range(n):
                cnt = sum(oracle.keep(m, j, n, t) for j in range(n))
                assert cnt == (m + 1 if m < cap else cap + 1)


def test_out_of_range_positions_are_masked(oracle):
    assert not oracle.keep(5, 0, 5, 0)
    assert not oracle.keep(0, 5, 5, 0)
    assert not oracle.keep(-1, 0, 5, 0)
    assert not oracle.keep(0, 0, 0, 0)


def test_targets_do_not_see_each_other(oracle):
    n, t = 12, 4
    cap = n - t
    for m in range(cap, n):
        for j in range(cap, n):
            assert oracle.keep(m, j, n, t) == (m == j)
        for j in range(cap):
            assert oracle.keep(m, j, n, t)


def test_more_targets_than_tokens_is_diagonal_only(oracle):
    for n in (1, 4, 9):
        for t in (n, n + 1, n + 7):
            for m in range(n):
                for j in range(n):
                    assert oracle.keep(m, j, n, t) == (m == j)


def test_prefix_rule_adds_exactly_the_upper_prefix_pairs(oracle):
    n, t, c = 20, 5, 6
    for m in range(n):
        for j in range(n):
            base = oracle.keep(m, j, n, t)
            with_ctx = oracle.keep(m, j, n, t, c, oracle.CTX_PREFIX)
            assert with_ctx == (base or j < c)
            if with_ctx and not base:
                assert m < j < c


def test_reference_rule_is_a_switch_on_key_zero(oracle):
    # with history present (cap > 0) the reference rule changes nothing under the causal mask;
    # with cap == 0 every key becomes visible; with cap < 0 nothing changes
    for n, t in ((9, 2), (9, 0), (5, 4)):
        for m in range(n):
            for j in range(n):
                assert oracle.keep(m, j, n, t, 8, oracle.CTX_REFCPP) == oracle.keep(m, j, n, t)
    n = 6
    for m in range(n):
        for j in range(n):
            assert oracle.keep(m, j, n, n, 3, oracle.CTX_REFCPP)
            assert oracle.keep(m, j, n, n + 2, 3, oracle.CTX_REFCPP) == (m == j)


@pytest.mark.parametrize("ctx", [0, 1, 8])
def test_pair_count_closed_form(oracle, ctx):
    for n in range(0, 41):
        for t in range(0, n + 1):
            if ctx > n - t:
                continue
            assert oracle.count_pairs(n, t, ctx) == oracle.pairs_closed_form(n, t, ctx)


def test_dense_mask_matches_scalar_mask(oracle):
    lengths = np.array([0, 6, 2, 9])
    targets = np.array([0, 2, 1, 3])
    N = 9
    for ctx in (0, 2):
        dense = oracle.keep_mask_dense(N, lengths, targets, ctx)
        for b in range(4):
            for m in range(N):
                for j in range(N):
                    assert dense[b, m, j] == oracle.keep(m, j, int(lengths[b]), int(targets[b]), ctx)


def test_workload_flop_model_matches_brute_force(oracle):
    from recir_amd.workloads import make_config

    wl = make_config(1)
    brute = sum(oracle.count_pairs(int(n), int(t)) for n, t in zip(wl.lengths, wl.num_targets))
    assert wl.pairs() == brute == 816
    assert wl.flops() == 208896
    wl2 = make_config(2)
    assert wl2.T == 39382 and wl2.pairs() == 28464549
    assert wl2.lengths[:4].tolist() == [1726 + 64, 1357 + 64, 1139 + 64, 722 + 64]
    wl4 = make_config(4)
    assert (wl4.lengths - 128).tolist() == [158, 128, 4705, 8064, 690, 8064, 128, 128]
    assert wl4.T == 23089


def test_semilocal_mask_forms_agree_exhaustively(oracle):
    """The "history key, near or full-tail row" form against the reference's clamped-id arithmetic
    (kjt_split_per_feature.cpp:639-674) for every (n, t, A, F, ctx, m, j) with n <= 18."""
    L = oracle.lib()
    for n in range(0, 19):
        for t in list(range(0, n + 1)) + [n + 2]:
            for A in (0, 1, 2, 3, 6, 40):
                for F in (0, 1, 3, 7, 40):
                    for ctx, mode in ((0, 0), (2, 0), (1, 1)):
                        for m in range(n):
                            for j in range(n):
                                a = L.hstu_oracle_keep_sl(m, j, n, t, ctx, mode, A, F)
                                b = L.hstu_oracle_keep_sl_clamp_id(m, j, n, t, ctx, mode, A, F)
                                assert a == b, (n, t, A, F, ctx, mode, m, j)


def test_semilocal_mask_matches_the_accelerator_kernels_form(oracle):
    """Third form, the one the reference's accelerator kernels use for the 256/256 shape
    (helion/jagged_hstu_attention.py:124-147): local | full | diagonal on the raw query index,
    valid when full_attn_size > 0 and targets do not exceed the length."""
    for n in (1, 5, 13, 30):
        for t in (0, 1, n // 3, n):
            hist_end = n - t
            for A in (1, 4, 9):
                for F in (1, 3, 12, 64):
                    full_start = hist_end - F
                    for m in range(n):
                        for j in range(n):
                            hk = j < hist_end
                            local = (m >= j) and (m - j <= A) and (m < full_start) and hk
                            full = (m >= j) and (m >= full_start) and hk
                            want = local or full or (m == j)
                            assert oracle.keep_sl(m, j, n, t, 0, 0, A, F) == want, (n, t, A, F, m, j)


def test_semilocal_reduces_to_causal_and_counts_rows(oracle):
    n, t = 23, 5
    cap = n - t
    for m in range(n):
        for j in range(n):
            # no window: full_attn_size alone changes nothing; a window at least as long as the history is causal
            assert oracle.keep_sl(m, j, n, t, 0, 0, 0, 7) == oracle.keep(m, j, n, t)
            assert oracle.keep_sl(m, j, n, t, 0, 0, n, 0) == oracle.keep(m, j, n, t)
    A, F = 4, 6
    for m in range(n):
        cnt = sum(oracle.keep_sl(m, j, n, t, 0, 0, A, F) for j in range(n))
        idm = min(m, cap)
        assert cnt == 1 + (idm if idm >= cap - F else min(idm, A))


def test_workload_pair_count_matches_brute_force_with_windows(oracle):
    from recir_amd.workloads import make_jagged

    rng = np.random.default_rng(3)
    for _ in range(60):
        B = int(rng.integers(1, 5))
        lengths = rng.integers(0, 28, size=B)
        targets = [int(rng.integers(0, l + 3)) for l in lengths]
        A, F, c = int(rng.choice([0, 1, 3, 7, 40])), int(rng.choice([0, 1, 4, 50])), int(rng.choice([0, 1, 3, 9]))
        wl = make_jagged(lengths, targets, 1, 4, 4, max_seq_len=40, alpha=1.0, contextual_seq_len=c,
                         max_attn_len=A, full_attn_size=F)
        want = sum(oracle.count_pairs_sl(int(n), int(t), c, 0, A, F) for n, t in zip(lengths, targets))
        assert wl.pairs() == want


def test_two_forms_of_the_noncausal_mask_agree_exhaustively(oracle):
    """Mask of a mask type other than "lower_triangular" (kjt_split_per_feature.cpp:650-671): the form
    that follows the reference line by line against the one said in words."""
    L = oracle.lib()
    for n in range(0, 21):
        for t in list(range(0, n + 1)) + [n + 1, n + 5]:
            for ctx, mode in ((0, 0), (3, 0), (1, 1)):
                for A, F in ((0, 0), (0, 3), (1, 0), (3, 0), (3, 2), (2, 50), (50, 1)):
                    for m in range(n):
                        for j in range(n):
                            a = L.hstu_oracle_keep_nc(m, j, n, t, ctx, mode, A, F)
                            b = L.hstu_oracle_keep_nc_clamp_id(m, j, n, t, ctx, mode, A, F)
                            assert a == b, (n, t, ctx, mode, A, F, m, j)


def test_noncausal_mask_properties(oracle):
    """What the reference's other branch comes to: without a window only the diagonal (and the
    contextual keys); with a window and no tail it is symmetric, every pair of targets is kept (they
    all stand at one position), and it contains the semi-local causal mask of the same window."""
    n, t = 14, 4
    for m in range(n):
        for j in range(n):
            assert oracle.keep_nc(m, j, n, t) == (m == j)
            assert oracle.keep_nc(m, j, n, t, 3, oracle.CTX_PREFIX) == (m == j or j < 3)
            for A in (1, 3, 20):
                k = oracle.keep_nc(m, j, n, t, 0, 0, A, 0)
                assert k == oracle.keep_nc(j, m, n, t, 0, 0, A, 0)
                assert k == (abs(min(m, n - t) - min(j, n - t)) <= A or m == j)
                if m >= n - t and j >= n - t:
                    assert k
                for F in (0, 2):
                    if oracle.keep_sl(m, j, n, t, 0, 0, A, F):
                        assert oracle.keep_nc(m, j, n, t, 0, 0, A, F)
    # the dispatch by mask type reaches the same functions
    assert oracle.keep_sl(2, 5, 9, 0, 0, 0, 3, 0, mask_type="full") and not oracle.keep_sl(2, 5, 9, 0, 0, 0, 3, 0)
    assert oracle.count_pairs_sl(9, 0, mask_type="full") == 9
