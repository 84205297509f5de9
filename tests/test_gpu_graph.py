"""The entry points under HIP graph capture: a forward (the entry point that allocates nothing, and the one
with a caller-owned workspace) and a backward are recorded once and replayed several times on fresh
values, with eager work and synchronisations between the replays; every replay must equal the eager
result of the same values bit for bit.  The library launches kernels only (its clears are fill kernels,
not runtime memsets), so the recorded graph holds nothing else."""
import ctypes

import pytest
import torch

from recir_amd import _lib
from recir_amd.workloads import make_jagged

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


class _Calls:
    """Static device buffers of one workload and the two C-ABI calls on them."""

    def __init__(self, lib, wl, dtype, code, with_rab_grad):
        dev = torch.device("cuda:0")
        self.lib, self.wl, self.code = lib, wl, code
        self.q, self.k, self.v = (t.to(dev, dtype) for t in (wl.q, wl.k, wl.v))
        self.dout = torch.randn_like(self.v)
        self.off, self.nt = wl.seq_offsets.to(dev), wl.num_targets.to(dev)
        self.rab = None if wl.rab is None else wl.rab.to(dev)
        T, H, Dqk = self.q.shape
        Dv = self.v.shape[2]
        self.dims = (T, wl.B, H, Dqk, Dv)
        self.tail = (wl.max_seq_len, wl.contextual_seq_len, wl.max_attn_len, wl.full_attn_size, wl.alpha, code, 0)
        self.drab = torch.empty_like(self.rab) if (with_rab_grad and self.rab is not None) else None
        need_f = lib.recir_hstu_attn_fwd_workspace_bytes(*self.dims, code)
        need_b = lib.recir_hstu_attn_bwd_workspace_bytes(*self.dims, code)
        if self.drab is not None:
            need_b += lib.recir_hstu_attn_bwd_rab_grad_workspace_bytes(H, wl.max_seq_len)
        self.ws_f = torch.empty(need_f, dtype=torch.uint8, device=dev)
        self.ws_b = torch.empty(need_b, dtype=torch.uint8, device=dev)

    def outputs(self):
        return dict(out=torch.empty_like(self.v), dq=torch.empty_like(self.q), dk=torch.empty_like(self.k),
                    dv=torch.empty_like(self.v), drab=None if self.drab is None else torch.empty_like(self.drab))

    def run(self, o, noalloc):
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        head = (_ptr(self.q), _ptr(self.k), _ptr(self.v), _ptr(o["out"]), _ptr(self.off), _ptr(self.nt), _ptr(self.rab),
                None, None, None, *self.dims, *self.tail)
        if noalloc:
            rc = self.lib.recir_hstu_attn_fwd_noalloc(*head, s)
        else:
            rc = self.lib.recir_hstu_attn_fwd(*head, _ptr(self.ws_f), self.ws_f.numel(), s)
        assert rc == 0, self.lib.recir_hstu_last_error().decode()
        rc = self.lib.recir_hstu_attn_bwd(_ptr(self.dout), _ptr(self.q), _ptr(self.k), _ptr(self.v), _ptr(o["dq"]), _ptr(o["dk"]),
                                          _ptr(o["dv"]), _ptr(o["drab"]), _ptr(self.off), _ptr(self.nt), _ptr(self.rab), None,
                                          *self.dims, *self.tail, _ptr(self.ws_b), self.ws_b.numel(), s)
        assert rc == 0, self.lib.recir_hstu_last_error().decode()


CASES = {
    # name: (Dqk, Dv, torch dtype, workload dtype, dtype code, bias, its gradient, entry point that allocates nothing)
    "head_dim_128_bf16_noalloc": (128, 128, torch.bfloat16, "bf16", _lib.DTYPE_BF16, False, False, True),
    "head_dim_128_bf16_bias_gradient": (128, 128, torch.bfloat16, "bf16", _lib.DTYPE_BF16, True, True, False),
    "head_dim_64_fp16_general_kernels": (64, 64, torch.float16, "fp16", _lib.DTYPE_FP16, False, False, True),
    "head_dim_32_fp32_general_kernels": (32, 48, torch.float32, "fp32", _lib.DTYPE_FP32, True, False, False),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_replays_of_a_captured_forward_and_backward_equal_the_eager_calls(case):
    dqk, dv, tdt, wdt, code, with_rab, rab_grad, noalloc = CASES[case]
    lib = _lib.load()
    wl = make_jagged([300, 129, 64, 1, 0, 517], [40, 129, 0, 0, 0, 6], 2, dqk, dv, max_seq_len=600, alpha=1.0 / dqk ** 0.5,
                     dtype=wdt, seed=3, with_rab=with_rab, rab_std=0.5, contextual_seq_len=2, tail_rows=5)
    c = _Calls(lib, wl, tdt, code, rab_grad)
    eager, graphed = c.outputs(), c.outputs()
    c.run(eager, noalloc)  # warm-up outside the capture (the first call of the no-allocation entry point looks up its scratch)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        c.run(graphed, noalloc)
    gen = torch.Generator(device="cuda").manual_seed(17)
    for rep in range(3):
        for t in (c.q, c.k, c.v, c.dout):  # fresh values in the buffers the graph reads: eager work between the replays
            t.copy_(torch.randn(t.shape, generator=gen, device=t.device).to(t.dtype))
        for o in graphed.values():
            if o is not None:
                o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        c.run(eager, noalloc)
        torch.cuda.synchronize()
        for name in ("out", "dq", "dk", "dv"):
            assert torch.equal(graphed[name].view(torch.uint8), eager[name].view(torch.uint8)), (case, rep, name)
        if rab_grad:
            # the head-dim-128 kernels sum the table's gradient in fixed point: the same bits every time
            assert torch.equal(graphed["drab"], eager["drab"]), (case, rep, "drab")
        assert torch.isfinite(graphed["out"].float()).all().item()
