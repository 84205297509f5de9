"""The operator inside RecIR's graph machinery: the swap of the reference's own source operator
(recir/lowering/op_swap.py:78-97 semantics) and the operator under ``torch.compile``
(recir/lowering/partial_lower.py:414-427 keeps a custom op with a Meta kernel inside the lowered region
and runs it from ``compile_fx`` output, :291-390).

The source operator is the reference's compiled C++ translation unit (``oracle/_ref``), loaded as a
library; none of the reference's Python is imported.  ``swap`` below restates what ``swap_ops`` does.
"""
import copy
import operator

import numpy as np
import pytest
import torch
import torch.fx as fx

from tests.parity_util import FP32_ATOL, FP32_RTOL, assert_bf16_close, expected_kernel


class Registry:
    """Same surface as recir.lowering.op_swap.OpSwapRegistry (register / swap_map)."""

    def __init__(self):
        self.swap_map = {}

    def register(self, source_op, replace_op):
        self.swap_map[source_op] = replace_op


def swap(gm, registry):
    """Retarget every call_function node whose target is in the registry; arguments untouched."""
    count = 0
    for node in list(gm.graph.nodes):
        if node.op == "call_function" and node.target in registry.swap_map:
            node.target = registry.swap_map[node.target]
            count += 1
    if count:
        gm.recompile()
    return count


def _reference_op():
    from oracle import hstu_oracle

    if not hstu_oracle.ref_available():
        pytest.skip("oracle/_ref/libkjt_ref.so not built (make -C oracle ref)")
    return hstu_oracle.ref_op()


def _graph_with_reference_node(N, alpha, ctx, max_attn_len=0, full_attn_size=0):
    """A graph as a trace of the third-party model leaves it: one node that calls the reference's
    ``hammer::triton_ragged_attention_fwd.default`` with its positional argument list, a getitem
    and a pointwise op after it."""
    src = torch.ops.hammer.triton_ragged_attention_fwd.default
    g = fx.Graph()
    q, k, v, off, nt = (g.placeholder(n) for n in ("q", "k", "v", "seq_offsets", "num_targets"))
    node = g.call_function(src, (N, alpha, q, k, v, off, "lower_triangular", nt, None, max_attn_len, ctx,
                                 full_attn_size, 0))
    out = g.call_function(operator.getitem, (node, 0))
    out = g.call_function(torch.mul, (out, 2.0))
    g.output(out)
    g.lint()
    return fx.GraphModule(torch.nn.Module(), g), node


def test_register_swaps_maps_the_reference_operator_and_swap_retargets_its_node():
    import recir_amd

    packet = _reference_op()
    reg = Registry()
    added = recir_amd.register_swaps(reg)
    assert added == 2 and len(reg.swap_map) == 2
    assert reg.swap_map[packet] is recir_amd.triton_ragged_attention_fwd
    assert reg.swap_map[packet.default] is recir_amd.triton_ragged_attention_fwd.default
    # argument for argument: the replacement has the schema of the operator it replaces
    src_args = [(a.name, str(a.type)) for a in packet.default._schema.arguments]
    dst_args = [(a.name, str(a.type)) for a in recir_amd.triton_ragged_attention_fwd.default._schema.arguments]
    assert src_args == dst_args
    assert [str(r.type) for r in packet.default._schema.returns] == \
        [str(r.type) for r in recir_amd.triton_ragged_attention_fwd.default._schema.returns]

    gm, node = _graph_with_reference_node(16, 0.25, 4)
    args_before = tuple(node.args)
    swapped = copy.deepcopy(gm)
    assert swap(swapped, reg) == 1
    new = [n for n in swapped.graph.nodes if n.op == "call_function"][0]
    assert new.target is recir_amd.triton_ragged_attention_fwd.default
    assert tuple(str(a) for a in new.args) == tuple(str(a) for a in args_before)
    assert "recir.triton_ragged_attention_fwd" in swapped.code
    # the original still runs the reference operator on the CPU
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(10, 2, 8, generator=g) for _ in range(3))
    off = torch.tensor([0, 6, 10])
    nt = torch.tensor([2, 1])
    assert gm(q, k, v, off, nt).shape == (10, 2, 8)
    # and the swapped graph traces with fake tensors (the Meta kernel the lowering asks for)
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        fq = torch.empty(10, 2, 8)
        out = swapped(fq, fq, fq, torch.empty(3, dtype=torch.int64), torch.empty(2, dtype=torch.int64))
    assert out.shape == (10, 2, 8)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["fp32_small_heads_ctx4", "bf16_d128_ctx4", "bf16_d128_semilocal"])
def test_swapped_graph_on_the_gpu_matches_the_original_graph_on_the_cpu(case):
    """The original graph runs the reference operator on CPU tensors, the swapped one the HIP operator
    on CUDA tensors: same numbers, including for contextual_seq_len > 1, where the reference's rule
    (keys whose target-clamped id is 0) differs from the prefix rule of ``hstu_jagged_attention_fwd``."""
    import recir_amd
    from recir_amd import _lib

    _reference_op()
    reg = Registry()
    recir_amd.register_swaps(reg)
    g = torch.Generator().manual_seed(17)
    if case == "fp32_small_heads_ctx4":
        lengths, targets, H, D, N, alpha, A, F = [7, 0, 12, 5], [2, 0, 12, 0], 2, 8, 16, 0.31, 0, 0
        dt = torch.float32
    elif case == "bf16_d128_ctx4":
        lengths, targets, H, D, N, alpha, A, F = [150, 64, 1, 200], [20, 64, 0, 7], 2, 128, 256, 1.0 / 128, 0, 0
        dt = torch.bfloat16
    else:
        lengths, targets, H, D, N, alpha, A, F = [300, 90], [30, 0], 2, 128, 320, 1.0 / 128, 48, 64
        dt = torch.bfloat16
    T = sum(lengths)
    q, k, v = (torch.randn(T, H, D, generator=g).to(dt).float() for _ in range(3))
    off = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int64)
    nt = torch.tensor(targets, dtype=torch.int64)
    gm, _ = _graph_with_reference_node(N, alpha, 4, A, F)
    want = gm(q, k, v, off, nt)  # reference operator, fp32 arithmetic on the (bf16-representable) values
    swapped = copy.deepcopy(gm)
    assert swap(swapped, reg) == 1
    dev = torch.device("cuda:0")
    got = swapped(q.to(dev, dt), k.to(dev, dt), v.to(dev, dt), off.to(dev), nt.to(dev))
    torch.cuda.synchronize()
    assert got.shape == want.shape  # no padding rows here: T == seq_offsets[-1]
    if dt == torch.float32:
        assert _lib.last_kernel() == expected_kernel(q.shape[2], v.shape[2], "fp32")
        np.testing.assert_allclose(got.cpu().numpy(), want.numpy(), rtol=FP32_RTOL, atol=FP32_ATOL)
    else:
        assert _lib.last_kernel().startswith("tiled_d128")
        assert_bf16_close(got, want.numpy(), f"swapped graph {case}")


def _attention_fn(N, alpha, nt_targets=True):
    def f(q, k, v, off, nt):
        q2 = q * 1.25  # pointwise producer
        out, _aux = torch.ops.recir.hstu_jagged_attention_fwd(N, alpha, q2, k, v, off, "lower_triangular", nt, None,
                                                              0, 0, 0)
        return torch.tanh(out.float()) * 3.0  # pointwise consumer

    return f


def _compiled_against_eager(backend):
    """pointwise -> attention -> pointwise under ``torch.compile(fullgraph=True, backend=...)``: no
    graph break; forward and gradients against eager.  An exception from the backend propagates."""
    import torch._dynamo as dynamo

    import recir_amd  # noqa: F401

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(5)
    lengths, targets, H, D, N = [200, 64, 130], [16, 0, 130], 2, 128, 256
    T = sum(lengths) + 3
    mk = lambda: torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    q, k, v = mk(), mk(), mk()
    off = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int64, device=dev)
    nt = torch.tensor(targets, dtype=torch.int64, device=dev)
    f = _attention_fn(N, 1.0 / 128)

    def run(fn):
        for t in (q, k, v):
            t.grad = None
        out = fn(q, k, v, off, nt)
        out.sum().backward()
        torch.cuda.synchronize()
        return out.detach().clone(), q.grad.clone(), k.grad.clone(), v.grad.clone()

    want = run(f)
    explanation = dynamo.explain(f)(q, k, v, off, nt)
    assert explanation.graph_break_count == 0 and explanation.graph_count == 1, str(explanation)
    dynamo.reset()
    got = run(torch.compile(f, fullgraph=True, backend=backend))
    dynamo.reset()
    for name, a, b in zip(("out", "dq", "dk", "dv"), got, want):
        if name == "out" or backend == "aot_eager":
            assert torch.equal(a, b), name
        else:
            # Inductor fuses tanh' * 3 * grad into one kernel whose fp32 rounding may differ from the
            # eager chain by an ulp before the bf16 cast; the attention gradients are then compared
            # to a tolerance of one bf16 ulp of the largest value instead of bit for bit
            assert (a.float() - b.float()).abs().max().item() <= 2 ** -7 * b.float().abs().max().item(), name
    assert got[0].abs().sum().item() > 0 and got[1].abs().sum().item() > 0


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_operator_under_torch_compile_inductor_fullgraph_forward_and_backward():
    """The operator is one opaque node with a Meta kernel and an autograd formula; Inductor generates
    code only for the pointwise operations around it.  No fallback: if Inductor raises, this fails."""
    _compiled_against_eager("inductor")


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_operator_under_torch_compile_aot_eager_fullgraph_forward_and_backward():
    """The same through AOTAutograd without code generation: bit for bit equal to eager."""
    _compiled_against_eager("aot_eager")


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_opcheck_of_the_forward_and_backward_operators():
    """torch.library.opcheck: schema, fake kernel, autograd registration and AOT dispatch of the
    operators (the checks RecIR's lowering relies on when it keeps the node opaque)."""
    import recir_amd  # noqa: F401

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(9)
    T, H, D, N = 70, 2, 128, 64
    mk = lambda grad: torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(dev).requires_grad_(grad)
    off = torch.tensor([0, 40, 40, 67], dtype=torch.int64, device=dev)
    nt = torch.tensor([5, 0, 27], dtype=torch.int64, device=dev)
    for op in (torch.ops.recir.hstu_jagged_attention_fwd.default, torch.ops.recir.triton_ragged_attention_fwd.default):
        args = (N, 0.01, mk(True), mk(True), mk(True), off, "lower_triangular", nt, None, 0, 2, 0)
        torch.library.opcheck(op, args)
    dout = mk(False)
    args = (dout, N, 0.01, mk(False), mk(False), mk(False), off, nt, None, 2)
    torch.library.opcheck(torch.ops.recir.hstu_jagged_attention_bwd.default, args)
    torch.library.opcheck(torch.ops.recir.triton_ragged_attention_bwd.default, args)
