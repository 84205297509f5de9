"""Writes the golden fixtures from the reference's own compiled C++ operator.

Run in the development container only (needs oracle/_ref/libkjt_ref.so, built from the upstream
checkout by `make -C oracle ref`):

    python tests/golden/make_golden.py            everything
    python tests/golden/make_golden.py noncausal  only the cases of a mask type other than the causal one

Outputs (data only):
  tests/golden/small_cases.npz   expected out[seq_offsets[B], H, Dv] per small case
  tests/golden/small_cases_bwd.npz  per small case, dq/dk/dv from torch autograd through the same
                                 operator for a seeded upstream gradient (the reference's own
                                 definition of its backward oracle, helion jagged_hstu_attention.py:260-280)
  tests/golden/noncausal_cases.npz, noncausal_cases_bwd.npz  the same two for the cases whose
                                 invalid_attn_mask_type is not "lower_triangular"
  tests/golden/config2.npz       config 2 (bf16-rounded inputs, fp32 arithmetic): per-sequence sums,
                                 abs-sums and 64 sampled rows
  tests/golden/config4.npz       same for the long skewed config 4

The reference operator takes contextual_seq_len as a boolean "key 0 is visible" switch
(kjt_split_per_feature.cpp:672-674); cases with ctx > 0 therefore pin the reference rule.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import hstu_oracle  # noqa: E402
from recir_amd.workloads import make_config  # noqa: E402
from tests.golden.cases import SMALL_CASES, build_inputs, fixture_file  # noqa: E402

SAMPLED_ROWS = 64


def run_ref(wl, scale, nt):
    return hstu_oracle.ref_attn_fwd(wl.q, wl.k, wl.v, wl.seq_offsets, nt, max_seq_len=wl.max_seq_len,
                                    alpha=wl.alpha, attn_scale=scale,
                                    contextual_seq_len=wl.contextual_seq_len,
                                    max_attn_len=wl.max_attn_len, full_attn_size=wl.full_attn_size,
                                    mask_type=wl.mask_type)


def run_ref_bwd(wl, scale, nt, dout):
    """(dq, dk, dv) by autograd through the reference operator; rows after seq_offsets[B] get no gradient."""
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (wl.q, wl.k, wl.v))
    out = hstu_oracle.ref_attn_fwd(q, k, v, wl.seq_offsets, nt, max_seq_len=wl.max_seq_len,
                                   alpha=wl.alpha, attn_scale=scale,
                                   contextual_seq_len=wl.contextual_seq_len,
                                   max_attn_len=wl.max_attn_len, full_attn_size=wl.full_attn_size,
                                   mask_type=wl.mask_type)
    out.backward(dout[: out.shape[0]])
    return q.grad, k.grad, v.grad


def sampled_rows(total_rows, seed=1234):
    rng = np.random.Generator(np.random.PCG64(seed))
    return np.sort(rng.choice(total_rows, size=min(SAMPLED_ROWS, total_rows), replace=False))


def checksum_fixture(config):
    wl = make_config(config)
    out = run_ref(wl, None, wl.num_targets).double()
    off = wl.seq_offsets.numpy()
    sums = np.array([out[off[b]:off[b + 1]].sum().item() for b in range(wl.B)])
    abss = np.array([out[off[b]:off[b + 1]].abs().sum().item() for b in range(wl.B)])
    rows = sampled_rows(int(off[-1]))
    return dict(seq_sum=sums, seq_abs_sum=abss, rows=rows, row_values=out[rows].float().numpy(),
                lengths=wl.lengths, T=np.int64(wl.T))


def main():
    torch.set_num_threads(os.cpu_count())
    only_noncausal = sys.argv[1:] == ["noncausal"]
    from tests.golden.cases import upstream_gradient  # noqa: E402

    fwd, bwd = {}, {}
    for name, case in SMALL_CASES.items():
        if only_noncausal and case["mask_type"] == "lower_triangular":
            continue
        wl, scale, nt = build_inputs(case)
        fwd.setdefault(fixture_file(case), {})[name] = run_ref(wl, scale, nt).numpy()
        print(name, fwd[fixture_file(case)][name].shape)
        if case["Dqk"] >= 128:
            continue  # keeps the fixture small; these shapes are compared with the live operator
        dq, dk, dv = run_ref_bwd(wl, scale, nt, upstream_gradient(case, wl))
        group = bwd.setdefault(fixture_file(case, backward=True), {})
        group[name + "/dq"], group[name + "/dk"], group[name + "/dv"] = dq.numpy(), dk.numpy(), dv.numpy()
    for fname, arrays in list(fwd.items()) + list(bwd.items()):
        np.savez_compressed(os.path.join(HERE, fname), **arrays)
    if only_noncausal:
        return
    for cfg in (2, 4):
        fx = checksum_fixture(cfg)
        np.savez_compressed(os.path.join(HERE, f"config{cfg}.npz"), **fx)
        print("config", cfg, fx["row_values"].shape)


if __name__ == "__main__":
    main()
