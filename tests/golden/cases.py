"""Definitions of the golden cases: inputs are regenerated from these seeds, never stored twice.

Shapes of the "ref_*" cases are the fixtures of the reference's own jagged-kernel tests
(recir/ops/pallas/tests/test_jagged_hstu_attention.py:163-203: lengths [7,3,9]; [0,6,2,0] with
targets [0,2,1,0]; every start residue [r,5] with targets [0,2]; [5,9] with targets [1,3], scale
0.31, inv_n 0.07; nine sequences [1]*8+[2]; heads 2, Dqk 8, Dv 6, inv_n 0.17, alpha 1/sqrt(8)).
Their values there come from a JAX PRNG that is not reproducible here, so the expected outputs in
the fixture come from the reference's compiled C++ operator on torch-seeded inputs instead.
"""
import math

SMALL_CASES = {}


def _add(name, lengths, targets, N, *, H=2, Dqk=8, Dv=6, alpha=None, attn_scale=0.17, ctx=0,
         per_token_scale=False, seed=0, tail_rows=0, no_targets=False, bf16_inputs=False,
         max_attn_len=0, full_attn_size=0, mask_type="lower_triangular"):
    SMALL_CASES[name] = dict(lengths=list(lengths), targets=list(targets), N=N, H=H, Dqk=Dqk, Dv=Dv,
                             alpha=(1.0 / math.sqrt(Dqk)) if alpha is None else alpha,
                             attn_scale=attn_scale, ctx=ctx, per_token_scale=per_token_scale,
                             seed=seed, tail_rows=tail_rows, no_targets=no_targets,
                             bf16_inputs=bf16_inputs, max_attn_len=max_attn_len,
                             full_attn_size=full_attn_size, mask_type=mask_type)


_add("ref_nonuniform_causal", [7, 3, 9], [0, 0, 0], 9)
_add("ref_targets_and_empty", [0, 6, 2, 0], [0, 2, 1, 0], 8)
for _r in range(8):
    _add(f"ref_residue_{_r}", [_r, 5], [0, 2], 8, seed=10 + _r)
_add("ref_block_invariance", [5, 9], [1, 3], 9, alpha=0.31, attn_scale=0.07)
_add("ref_nine_sequences", [1] * 8 + [2], [0] * 9, 2)
_add("ref_bwd_shape_3_5", [3, 5], [0, 2], 8)
_add("smoke_config1", [20] * 4, [4] * 4, 20, H=2, Dqk=32, Dv=32, alpha=1.0 / 32, attn_scale=None)
_add("no_targets_tensor", [7, 3, 9], [0, 0, 0], 9, no_targets=True, attn_scale=None)
_add("all_targets", [6, 4], [6, 4], 8)
_add("targets_exceed_length", [5, 3], [7, 3], 8)
_add("per_token_scale", [7, 3, 9], [2, 1, 3], 9, per_token_scale=True)
_add("tail_rows", [7, 3, 9], [2, 0, 1], 9, tail_rows=5)
_add("ctx1", [7, 3, 9], [2, 0, 1], 9, ctx=1)
_add("ctx8_reference_rule", [12, 3, 9, 4], [2, 0, 1, 4], 12, ctx=8)
# shapes that exercise the tiled head-dim-128 kernel: several key tiles, targets that straddle a
# tile boundary, a one-token and an empty sequence, tail rows
_add("d128_mixed", [130, 64, 257, 1, 0, 200], [3, 64, 70, 1, 0, 0], 300, H=2, Dqk=128, Dv=128,
     alpha=1.0 / 128, attn_scale=None, tail_rows=3, bf16_inputs=True)
_add("d128_ctx_refrule", [150, 70, 33], [20, 70, 0], 256, H=1, Dqk=128, Dv=128, alpha=1.0 / 128,
     attn_scale=0.01, ctx=4, bf16_inputs=True, seed=3)
# semi-local mask of the reference operator (kjt_split_per_feature.cpp:654-668): window only, window
# plus full-attention tail, a tail longer than the history, targets, the contextual switch, and
# head-dim-128 shapes whose windows cut through key tiles
_add("sl_window_only", [12, 3, 9, 20], [2, 0, 1, 5], 20, max_attn_len=3, seed=40)
_add("sl_window_and_tail", [12, 3, 9, 20], [2, 0, 1, 5], 20, max_attn_len=3, full_attn_size=4, seed=41)
_add("sl_tail_exceeds_history", [7, 3, 9], [2, 3, 0], 9, max_attn_len=2, full_attn_size=50, seed=42)
_add("sl_ctx_refrule", [10, 6, 1], [3, 6, 0], 10, max_attn_len=2, full_attn_size=2, ctx=1, seed=43)
_add("sl_full_size_without_window", [7, 3, 9], [1, 0, 2], 9, max_attn_len=0, full_attn_size=3, seed=44)
_add("d128_semilocal", [300, 130, 64, 257, 1], [10, 0, 64, 30, 0], 320, H=2, Dqk=128, Dv=128, alpha=1.0 / 128,
     attn_scale=None, tail_rows=2, bf16_inputs=True, max_attn_len=70, full_attn_size=40, seed=45)
_add("d128_semilocal_window_only", [260, 200], [0, 33], 300, H=1, Dqk=128, Dv=128, alpha=1.0 / 128,
     attn_scale=0.02, bf16_inputs=True, max_attn_len=64, seed=46)
# A mask type other than "lower_triangular" (kjt_split_per_feature.cpp:650-660: absolute distances):
# the diagonal alone without a window, a window either way round, window plus tail, targets beyond
# the length, the contextual switch, and head dim 128 in bf16.  Their expected outputs are kept in
# files of their own (fixture_file).
_add("nc_diagonal_only", [7, 3, 9], [2, 0, 1], 9, mask_type="full", seed=60)
_add("nc_window", [12, 3, 9, 20], [2, 0, 1, 5], 20, max_attn_len=3, mask_type="full", seed=61)
_add("nc_window_and_tail", [12, 3, 9, 20], [2, 0, 1, 5], 20, max_attn_len=3, full_attn_size=4, mask_type="full", seed=62)
_add("nc_tail_exceeds_history", [7, 3, 9], [2, 3, 0], 9, max_attn_len=2, full_attn_size=50, mask_type="full", seed=63)
_add("nc_targets_exceed_length", [5, 3, 6], [7, 3, 0], 8, max_attn_len=1, full_attn_size=2, mask_type="full", seed=64)
_add("nc_ctx_refrule", [10, 6, 1], [3, 6, 0], 10, max_attn_len=2, full_attn_size=2, ctx=1, mask_type="full", seed=65)
_add("nc_ctx_without_window", [10, 6, 1], [3, 6, 0], 10, ctx=1, per_token_scale=True, mask_type="upper_triangular", seed=66)
_add("nc_d128", [150, 70, 33, 1, 0], [20, 70, 0, 0, 0], 256, H=2, Dqk=128, Dv=128, alpha=1.0 / 128, attn_scale=0.01,
     bf16_inputs=True, max_attn_len=40, full_attn_size=16, tail_rows=2, mask_type="full", seed=67)


def fixture_file(case, backward=False):
    """Name of the .npz that holds the expected output (or gradients) of a case."""
    stem = "small_cases" if case["mask_type"] == "lower_triangular" else "noncausal_cases"
    return stem + ("_bwd.npz" if backward else ".npz")


def build_inputs(case):
    """(workload, attn_scale tensor or None, num_targets tensor or None) for a case dict."""
    import torch

    from recir_amd.workloads import make_jagged

    wl = make_jagged(case["lengths"], case["targets"], case["H"], case["Dqk"], case["Dv"],
                     max_seq_len=case["N"], alpha=case["alpha"],
                     dtype="bf16" if case["bf16_inputs"] else "fp32", seed=case["seed"],
                     contextual_seq_len=case["ctx"], tail_rows=case["tail_rows"],
                     max_attn_len=case["max_attn_len"], full_attn_size=case["full_attn_size"],
                     mask_type=case["mask_type"])
    if case["per_token_scale"]:
        g = torch.Generator().manual_seed(1000 + case["seed"])
        scale = torch.rand(wl.T, generator=g) * 0.5 + 0.05
    elif case["attn_scale"] is None:
        scale = None
    else:
        scale = torch.tensor(case["attn_scale"], dtype=torch.float32)
    nt = None if case["no_targets"] else wl.num_targets
    return wl, scale, nt


def upstream_gradient(case, wl):
    """Seeded upstream gradient dout [T,H,Dv] of a case (bf16-representable when the inputs are)."""
    import torch

    g = torch.Generator().manual_seed(7000 + case["seed"])
    dout = torch.randn(wl.T, wl.H, wl.v.shape[2], generator=g)
    if case["bf16_inputs"]:
        dout = dout.to(torch.bfloat16).float()
    return dout
