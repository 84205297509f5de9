"""The forward entry point that allocates nothing (``recir_hstu_attn_fwd_noalloc``) against the
entry point with a caller-owned workspace (``recir_hstu_attn_fwd``), both called through the C ABI.

Two calls in a row share the library's built-in scratch array; the second has a smaller input, so
anything the first call left behind lies beyond what the second one writes.  Outputs must be equal
bit for bit: the two entry points run the same kernels on the same work lists.
"""
import ctypes

import numpy as np
import pytest
import torch

from recir_amd import _lib
from recir_amd.workloads import make_jagged

pytestmark = pytest.mark.gpu


def _call(lib, wl, *, noalloc, stream=None):
    dev = torch.device("cuda:0")
    q = wl.q.to(dev, torch.bfloat16)
    k = wl.k.to(dev, torch.bfloat16)
    v = wl.v.to(dev, torch.bfloat16)
    off = wl.seq_offsets.to(dev)
    nt = wl.num_targets.to(dev)
    rab = None if wl.rab is None else wl.rab.to(dev)
    T, H, D = q.shape
    B = nt.shape[0]
    out = torch.full((T, H, D), float("nan"), dtype=torch.bfloat16, device=dev)
    ptr = lambda t: ctypes.c_void_p(0 if t is None else t.data_ptr())
    head = (ptr(q), ptr(k), ptr(v), ptr(out), ptr(off), ptr(nt), ptr(rab), None, None, None,
            T, B, H, D, D, wl.max_seq_len, wl.contextual_seq_len, wl.max_attn_len, wl.full_attn_size,
            wl.alpha, _lib.DTYPE_BF16, 0)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        rc = lib.recir_hstu_attn_fwd_noalloc(*head, s)
    else:
        need = lib.recir_hstu_attn_fwd_workspace_bytes(T, B, H, D, D, _lib.DTYPE_BF16)
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        rc = lib.recir_hstu_attn_fwd(*head, ptr(ws), need, s)
    assert rc == 0, lib.recir_hstu_last_error().decode()
    torch.cuda.synchronize()
    return out


def _workloads():
    rng = np.random.Generator(np.random.PCG64(11))
    big_len = rng.integers(200, 900, size=12)
    big = make_jagged(big_len, np.minimum(big_len // 4, 40), 4, 128, 128, max_seq_len=1024, alpha=1 / 128,
                      dtype="bf16", seed=5, tail_rows=37, name="noalloc_big")
    small_len = np.array([130, 1, 64, 257])
    small = make_jagged(small_len, [3, 0, 64, 20], 2, 128, 128, max_seq_len=512, alpha=1 / 128,
                        dtype="bf16", seed=6, contextual_seq_len=4, with_rab=True, tail_rows=5,
                        name="noalloc_small")
    return big, small


def test_noalloc_entry_matches_workspace_entry_on_two_calls_in_a_row():
    lib = _lib.load()
    big, small = _workloads()
    for wl in (big, small):  # the second, smaller call reuses the scratch the first one filled
        print(f"[noalloc] {wl.name}: T={wl.T} B={wl.B} H={wl.H}", flush=True)
        got = _call(lib, wl, noalloc=True)
        want = _call(lib, wl, noalloc=False)
        assert lib.recir_hstu_last_kernel().decode().startswith("tiled_d128_bf16")
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), wl.name
        end = int(wl.seq_offsets[-1])
        assert not got[end:].float().abs().any().item()
        assert torch.isfinite(got.float()).all().item()


def test_noalloc_entry_rejects_what_does_not_fit_and_plan_reuse():
    lib = _lib.load()
    # sizes whose work lists exceed the built-in scratch: rejected before any launch or pointer use
    T = 128 * 20000
    assert lib.recir_hstu_attn_fwd_workspace_bytes(T, 1, 4, 128, 128, _lib.DTYPE_BF16) > _lib.NOALLOC_SCRATCH_BYTES
    rc = lib.recir_hstu_attn_fwd_noalloc(8, 8, 8, 8, 8, None, None, None, None, None, T, 1, 4, 128, 128, 2048, 0, 0, 0,
                                         1.0, _lib.DTYPE_BF16, 0, None)
    assert rc == -3 and "exceed the built-in scratch" in lib.recir_hstu_last_error().decode()
    rc = lib.recir_hstu_attn_fwd_noalloc(8, 8, 8, 8, 8, None, None, None, None, None, 256, 1, 4, 128, 128, 2048, 0, 0, 0,
                                         1.0, _lib.DTYPE_BF16, _lib.FLAG_REUSE_PLAN, None)
    assert rc == -1 and "REUSE_PLAN" in lib.recir_hstu_last_error().decode()
