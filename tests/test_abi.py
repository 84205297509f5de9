"""The C-ABI library: it loads without a GPU, exports every symbol the header declares, rejects bad
arguments before any launch, and the host-side operator surface validates like the reference's."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    from recir_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        from recir_amd.build import build_library

        build_library()
    return _lib.load()


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "recir_hstu.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(recir_hstu_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_are_exported(lib):
    from recir_amd import _lib

    declared = _declared_symbols()
    assert declared == sorted(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_jagged_header_symbols_are_exported(lib):
    from recir_amd import _lib

    text = open(os.path.join(ROOT, "include", "recir_jagged.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    declared = sorted(set(re.findall(r"\b(recir_[a-z0-9_]+)\s*\(", text)))
    assert declared == sorted(_lib.JAGGED_EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name
    # argument rules are checked before any launch (no GPU needed)
    assert lib.recir_concat_2d_jagged(8, 8, 8, None, None, 1, 1, 1, 1, 1, 16, 0, 0, 0, None) < 0
    assert "at least one input must be jagged" in lib.recir_hstu_last_error().decode()
    assert lib.recir_jagged_to_padded_dense(8, 8, 8, 4, 1, 4, 0, 2, 0, 0, None) < 0
    assert "row_bytes" in lib.recir_hstu_last_error().decode()


def test_abi_version(lib):
    assert lib.recir_hstu_abi_version() == 6


def test_workspace_size_is_host_arithmetic(lib):
    # a 64-byte header plus 8 per-XCD lists of 32-byte items, each list able to hold every
    # (sequence, query tile, head) item: (ceil(T/128) + B) * H of them
    assert lib.recir_hstu_attn_fwd_workspace_bytes(39382, 32, 4, 128, 128, 0) == 64 + 32 * (308 + 32) * 4 * 8
    assert lib.recir_hstu_attn_fwd_workspace_bytes(0, 0, 1, 8, 8, 1) == 64
    assert lib.recir_hstu_attn_fwd_workspace_bytes(-1, 0, 1, 8, 8, 1) == 0


@pytest.mark.parametrize("kw,needle", [
    (dict(T=-1), "negative size"),
    (dict(H=0), "must be positive"),
    (dict(Dv=0), "must be positive"),
    (dict(N=0), "max_seq_len"),
    (dict(ctx=-2), "contextual_seq_len"),
    (dict(dtype=9), "unknown dtype"),
    (dict(q=None), "non-null"),
    (dict(off=None), "seq_offsets"),
    (dict(dtype=2), "q_scale"),
    (dict(A=-1), "max_attn_len and full_attn_size"),
])
def test_invalid_arguments_are_rejected_before_launch(lib, kw, needle):
    a = dict(q=8, k=8, v=8, out=8, off=8, T=4, B=1, H=1, Dqk=8, Dv=8, N=4, ctx=0, dtype=1, A=0, F=0)
    a.update(kw)
    rc = lib.recir_hstu_attn_fwd(a["q"], a["k"], a["v"], a["out"], a["off"], None, None, None, None, None,
                                 a["T"], a["B"], a["H"], a["Dqk"], a["Dv"], a["N"], a["ctx"], a["A"], a["F"], 1.0,
                                 a["dtype"], 0, None, 0, None)
    assert rc < 0
    assert needle in lib.recir_hstu_last_error().decode()


@pytest.mark.parametrize("kw,needle", [
    (dict(T=-1), "negative size"),
    (dict(H=0), "must be positive"),
    (dict(N=0), "max_seq_len"),
    (dict(F=-1), "max_attn_len and full_attn_size"),
    (dict(dtype=2), "bf16, fp16 and fp32"),
    (dict(dq=None), "non-null"),
    (dict(off=None), "seq_offsets"),
])
def test_backward_invalid_arguments_are_rejected_before_launch(lib, kw, needle):
    a = dict(dout=8, q=8, k=8, v=8, dq=8, dk=8, dv=8, off=8, T=4, B=1, H=1, Dqk=8, Dv=8, N=4, ctx=0, dtype=1, A=0, F=0)
    a.update(kw)
    rc = lib.recir_hstu_attn_bwd(a["dout"], a["q"], a["k"], a["v"], a["dq"], a["dk"], a["dv"], None, a["off"], None,
                                 None, None, a["T"], a["B"], a["H"], a["Dqk"], a["Dv"], a["N"], a["ctx"], a["A"], a["F"],
                                 1.0, a["dtype"], 0, None, 0, None)
    assert rc < 0
    assert needle in lib.recir_hstu_last_error().decode()


def test_backward_fake_kernel_and_autograd_wiring():
    """The backward operator traces with fake tensors, and the forward operator has an autograd
    formula that routes q, k, v gradients through it."""
    import recir_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(10, 2, 8, dtype=torch.bfloat16, requires_grad=True)
        v = torch.empty(10, 2, 6, dtype=torch.bfloat16, requires_grad=True)
        off = torch.empty(3, dtype=torch.int64)
        dq, dk, dv = torch.ops.recir.hstu_jagged_attention_bwd(torch.empty_like(v), 8, 0.5, q, q, v, off,
                                                               None, None, 0)
        assert dq.shape == q.shape and dk.shape == q.shape and dv.shape == v.shape
        out, _ = torch.ops.recir.hstu_jagged_attention_fwd(8, 0.5, q, q, v, off, "lower_triangular",
                                                          None, None, 0, 0, 0)
        assert out.requires_grad
        out.sum().backward()
        assert q.grad.shape == q.shape and v.grad.shape == v.shape


def test_empty_input_is_ok_without_launch(lib):
    rc = lib.recir_hstu_attn_fwd(None, None, None, None, None, None, None, None, None, None,
                                 0, 0, 2, 8, 8, 4, 0, 0, 0, 1.0, 1, 0, None, 0, None)
    assert rc == 0


def test_cpu_tensors_fail_loudly():
    import recir_amd

    q = torch.zeros(4, 1, 8)
    off = torch.tensor([0, 4])
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        recir_amd.jagged_hstu_attention(q, q, q, off, max_seq_len=4)


def test_index_tensors_follow_the_values_and_value_tensors_on_another_device_raise():
    """No host pointer may reach a kernel: offsets and target counts are moved to the device of q
    (the reference accepts them anywhere, recir/ops/kjt_split_per_feature.cpp:623-626), value tensors
    elsewhere are an error raised before any launch.  Nothing here touches a GPU."""
    from recir_amd import jagged, ops

    off = torch.tensor([0, 3, 5], dtype=torch.int64)
    nt = torch.tensor([1, 0], dtype=torch.int32)
    meta = torch.device("meta")
    o, t, flags = ops._index_tensors(off, nt, meta)
    assert o.device == meta and t.device == meta and t.dtype == torch.int64 and flags == 0
    o, t, flags = ops._index_tensors(off.int(), None, meta)
    assert o.device == meta and t is None and flags == ops._lib.FLAG_OFFSETS_I32
    o, _ = jagged._offsets(off, dev=meta)
    assert o.device == meta
    gpu = torch.device("cuda:0")  # only a name here: nothing is allocated on it
    with pytest.raises(ValueError, match="v is on cpu, q on cuda:0"):
        ops._check_same_device(gpu, k=None, v=torch.zeros(1))
    with pytest.raises(ValueError, match="timestamps is on cpu"):
        jagged._same_device(gpu, pos_embeddings=None, timestamps=torch.zeros(1))
    ops._check_same_device(torch.device("cpu"), k=torch.zeros(1), v=None)


def test_shape_errors_match_reference_messages():
    # recir/ops/pallas/tests/test_jagged_hstu_attention.py:679-690 ("shape [B]") and the validator
    # at recir/ops/pallas/jagged_hstu_attention.py:1498-1515
    import recir_amd

    q = torch.zeros(5, 2, 8)
    v = torch.zeros(5, 2, 6)
    off = torch.tensor([0, 3, 5])
    with pytest.raises(ValueError, match=r"shape \[B\]"):
        recir_amd.jagged_hstu_attention(q, q, v, off, torch.zeros(3, dtype=torch.int64), max_seq_len=4)
    with pytest.raises(ValueError, match=r"shape \[T, H, D\]"):
        recir_amd.jagged_hstu_attention(q[0], q, v, off, max_seq_len=4)
    with pytest.raises(ValueError, match="share packed-token and head"):
        recir_amd.jagged_hstu_attention(q, q, v[:4], off, max_seq_len=4)
    with pytest.raises(ValueError, match="feature dimension"):
        recir_amd.jagged_hstu_attention(q, q[:, :, :4], v, off, max_seq_len=4)
    with pytest.raises(ValueError, match=r"shape \[B \+ 1\]"):
        recir_amd.jagged_hstu_attention(q, q, v, off[:1], max_seq_len=4)
    with pytest.raises(ValueError, match="max_seq_len must be positive"):
        recir_amd.jagged_hstu_attention(q, q, v, off, max_seq_len=0)


def test_fake_kernel_and_schema():
    """The operator traces with fake tensors (the requirement of recir/lowering/partial_lower.py:
    414-427) and keeps the argument list of hammer::triton_ragged_attention_fwd
    (recir/ops/kjt_split_per_feature.cpp:780-783) plus a trailing optional rab."""
    import recir_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode

    schema = str(torch.ops.recir.hstu_jagged_attention_fwd.default._schema)
    want = ("int N, float alpha, Tensor q, Tensor k, Tensor v, Tensor seq_offsets, "
            "str invalid_attn_mask_type, Tensor? num_targets, Tensor? attn_scale, int max_attn_len, "
            "int contextual_seq_len, int full_attn_size, int num_softmax_heads=0")
    assert want in schema and schema.endswith("Tensor? rab=None) -> (Tensor, Tensor)")
    with FakeTensorMode():
        q = torch.empty(10, 2, 8, dtype=torch.bfloat16)
        v = torch.empty(10, 2, 6, dtype=torch.bfloat16)
        off = torch.empty(3, dtype=torch.int64)
        out, aux = torch.ops.recir.hstu_jagged_attention_fwd(8, 0.5, q, q, v, off, "lower_triangular",
                                                            None, None, 0, 0, 0)
        assert out.shape == (10, 2, 6) and out.dtype == torch.bfloat16
        assert aux.shape == (1,) and aux.dtype == torch.float32


def test_every_registered_operator_has_a_meta_kernel():
    """RecIR's lowering keeps a custom operator inside a lowered region only if FakeTensorMode can run
    it; its predicate (recir/lowering/lowering_utils.py:19-27) is the computed dispatch table's entry
    for the Meta key.  Evaluated here for every operator this package defines in ``recir::``."""
    import recir_amd  # noqa: F401

    names = [n for n in torch._C._dispatch_get_all_op_names() if n.startswith("recir::")]
    # the attention family, the quantiser and the jagged neighbours
    for must in ("recir::hstu_jagged_attention_fwd", "recir::hstu_jagged_attention_bwd",
                 "recir::hstu_jagged_attention_bwd_rab", "recir::triton_ragged_attention_fwd",
                 "recir::triton_ragged_attention_bwd", "recir::hstu_jagged_attention_fp8_fwd",
                 "recir::hstu_quantize_e4m3_per_head", "recir::concat_2d_jagged", "recir::split_2d_jagged"):
        assert must in names, must
    assert len(names) >= 12, names
    for name in names:
        assert torch._C._dispatch_has_computed_kernel_for_dispatch_key(name, "Meta"), name


def test_fp8_region_follows_the_contextual_rule_of_the_matched_operator():
    """A region cut around ``recir::triton_ragged_attention_fwd`` (the drop-in for the reference's
    operator, whose contextual rule is recir/ops/kjt_split_per_feature.cpp:672-674) is rewritten to
    the reference-rule fp8 entry, one around ``recir::hstu_jagged_attention_fwd`` to the prefix-rule
    one; the fp8 operator's schema carries the switch."""
    import torch.fx as fx
    from torch.fx.experimental.proxy_tensor import make_fx

    import recir_amd

    assert "bool reference_contextual_rule=False" in str(torch.ops.recir.hstu_jagged_attention_fp8_fwd.default._schema)
    for op, via in ((recir_amd.triton_ragged_attention_fwd.default, recir_amd.attention_via_fp8_reference_rule),
                    (recir_amd.hstu_jagged_attention_fwd.default, recir_amd.attention_via_fp8)):
        def f(q, k, v, off, nt):
            return op(16, 0.25, q, k, v, off, "lower_triangular", nt, None, 0, 4, 0)[0]

        q, k, v = (torch.empty(12, 2, 128, dtype=torch.bfloat16) for _ in range(3))
        gm = make_fx(f, tracing_mode="fake")(q, k, v, torch.empty(3, dtype=torch.int64), torch.empty(2, dtype=torch.int64))
        node = next(n for n in gm.graph.nodes if recir_amd.hstu_attention_matcher(n))
        region = fx.Graph()
        env = {a: region.placeholder(a.name) for a in node.args if isinstance(a, fx.Node)}
        region.output(region.node_copy(node, lambda n: env[n]))
        run = recir_amd.fp8_attention_region(fx.GraphModule(torch.nn.Module(), region))
        calls = [n for n in run.gm.graph.nodes if n.op == "call_function" and callable(n.target)
                 and getattr(n.target, "__module__", "") == "recir_amd.ops"]
        assert [c.target for c in calls] == [via]
        assert calls[0].args[10] == 4  # contextual_seq_len travels unchanged
        # traces with fake tensors end to end (quantiser and fp8 operator both have Meta kernels)
        from torch._subclasses.fake_tensor import FakeTensorMode

        with FakeTensorMode():
            qf = torch.empty(12, 2, 128, dtype=torch.bfloat16)
            out = via(16, 0.25, qf, qf, qf, torch.empty(3, dtype=torch.int64), "lower_triangular",
                      torch.empty(2, dtype=torch.int64), None, 0, 4, 0)[0]
            assert out.shape == (12, 2, 128)


def test_swap_registry_retargets_a_traced_node():
    """swap_ops rewrites node.target only (recir/lowering/op_swap.py:78-97): the replacement must
    accept the source operator's positional arguments unchanged."""
    import recir_amd

    lib = torch.library.Library("hammer_test_src", "DEF")
    lib.define("triton_ragged_attention_fwd(int N, float alpha, Tensor q, Tensor k, Tensor v, "
               "Tensor seq_offsets, str invalid_attn_mask_type, Tensor? num_targets, Tensor? attn_scale, "
               "int max_attn_len, int contextual_seq_len, int full_attn_size, int num_softmax_heads=0) "
               "-> (Tensor, Tensor)")

    @torch.library.register_fake("hammer_test_src::triton_ragged_attention_fwd")
    def _fake(N, alpha, q, k, v, off, mt, nt, sc, a, b, c, d=0):
        return v.new_empty(v.shape), v.new_empty((1,), dtype=torch.float32)

    src = torch.ops.hammer_test_src.triton_ragged_attention_fwd.default

    def f(q, k, v, off):
        return src(8, 0.5, q, k, v, off, "lower_triangular", None, None, 0, 0, 0)[0]

    from torch.fx.experimental.proxy_tensor import make_fx

    q = torch.empty(10, 2, 8, dtype=torch.bfloat16)
    gm = make_fx(f, tracing_mode="fake")(q, q, q, torch.empty(3, dtype=torch.int64))
    swapped = 0
    for node in gm.graph.nodes:  # what swap_ops does
        if node.op == "call_function" and node.target is src:
            node.target = recir_amd.hstu_jagged_attention_fwd.default
            swapped += 1
    gm.recompile()
    assert swapped == 1
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        qq = torch.empty(10, 2, 8, dtype=torch.bfloat16)
        out = gm(qq, qq, qq, torch.empty(3, dtype=torch.int64))
    assert out.shape == (10, 2, 8)


def test_register_swaps_fills_a_registry():
    """Two mappings (overload packet and ``.default``) once the reference's operator is in the process,
    none before; tests/test_swap_wiring.py runs a swapped graph."""
    import recir_amd
    from oracle import hstu_oracle

    class Registry:  # same surface as recir.lowering.op_swap.OpSwapRegistry.register
        def __init__(self):
            self.map = {}

        def register(self, source_op, replace_op):
            self.map[source_op] = replace_op

    if not hstu_oracle.ref_available():
        reg = Registry()
        assert recir_amd.register_swaps(reg) == 0 and not reg.map
        return
    src = hstu_oracle.ref_op()
    reg = Registry()
    assert recir_amd.register_swaps(reg) == 2
    assert reg.map == {src: recir_amd.triton_ragged_attention_fwd, src.default: recir_amd.triton_ragged_attention_fwd.default}


def _attention_graph():
    """A traced graph with one attention node, a getitem and a cast after it, plus the region a
    single-node match extracts from it (placeholders for the node's tensor inputs, constants inside),
    as recir/region_transforms/core.py builds it for inference_swap.py:293-307."""
    import torch.fx as fx

    import recir_amd
    from torch.fx.experimental.proxy_tensor import make_fx

    op = recir_amd.hstu_jagged_attention_fwd.default

    def f(q, k, v, off, nt):
        out, _aux = op(16, 0.25, q, k, v, off, "lower_triangular", nt, None, 0, 0, 0)
        return out.float() * 2.0

    q, k, v = (torch.empty(12, 2, 128, dtype=torch.bfloat16) for _ in range(3))
    gm = make_fx(f, tracing_mode="fake")(q, k, v, torch.empty(3, dtype=torch.int64), torch.empty(2, dtype=torch.int64))
    matched = [n for n in gm.graph.nodes if recir_amd.hstu_attention_matcher(n)]
    assert len(matched) == 1
    node = matched[0]
    region = fx.Graph()
    env = {}
    for a in node.args:
        if isinstance(a, fx.Node):
            env[a] = region.placeholder(a.name)
    new = region.node_copy(node, lambda n: env[n])
    region.output(new)
    return gm, node, fx.GraphModule(torch.nn.Module(), region)


def test_fp8_region_factory_rewrites_the_matched_region():
    """Matcher and factory of the training-to-inference swap: the factory's callable keeps the
    region's inputs and constants, runs the fp8 entry point in place of the attention node, can be
    pickled (its target is a module-level function), and has no CPU path."""
    import pickle

    import recir_amd

    gm, node, region_gm = _attention_graph()
    assert not any(recir_amd.hstu_attention_matcher(n) for n in gm.graph.nodes if n is not node)
    run = recir_amd.fp8_attention_region(region_gm)
    assert run.__name__ == "fp8_attention_region"  # usable as a call_function target
    calls = [n for n in run.gm.graph.nodes if n.op == "call_function"]
    assert len(calls) == 1 and calls[0].target is recir_amd.attention_via_fp8
    assert calls[0].args[0] == 16 and calls[0].args[1] == 0.25 and calls[0].args[6] == "lower_triangular"
    assert [n.op for n in run.gm.graph.nodes].count("placeholder") == 5
    # the region handed in is left as it was
    assert any(recir_amd.hstu_attention_matcher(n) for n in region_gm.graph.nodes)
    assert b"attention_via_fp8" in pickle.dumps(run)
    q = torch.zeros(12, 2, 128, dtype=torch.bfloat16)
    with pytest.raises((NotImplementedError, RuntimeError), match="no CPU implementation"):
        run(q, q, q, torch.tensor([0, 5, 12]), torch.tensor([1, 2]))
    with pytest.raises(ValueError, match="no HSTU attention node"):
        import torch.fx as fx

        g = fx.Graph()
        x = g.placeholder("x")
        g.output(x)
        recir_amd.fp8_attention_region(fx.GraphModule(torch.nn.Module(), g))
