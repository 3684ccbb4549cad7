"""The verify path's torch custom operators (batchspec_amd/ops.py) trace into one graph.

BatchSpec compiles its forward (batchspec/backends/standard_engine.py:104-106,
batchspec/backends/mtp_engine.py:165-169) and calls attention and the KV update as
registered operators (batchspec/models/mtp_model.py:82-84,
batchspec/models/modules/attention/mtp.py:82-93).  On the CPU, with a dynamo backend that
runs the captured graph under fake tensors (no kernel runs), these tests show that a
layer of update_kv + attention and both acceptance operators compile with
fullgraph=True (no graph break) and that the fake implementations give the shapes and
dtypes of the real ones."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import batchspec_amd as bsx
from batchspec_amd import ops


class _Unrun:
    def run(self, q, kv_cache):  # the fake implementation stands in; never called
        raise AssertionError("the real operator ran")


def _fake_backend(graphs):
    def backend(gm, example_inputs):
        graphs.append(gm)

        def run(*args):
            with FakeTensorMode(allow_non_fake_inputs=True):
                return gm(*args)
        return run
    return backend


def _i32(*x):
    return torch.tensor(x, dtype=torch.int32)


def test_layer_of_update_kv_and_attention_is_one_graph():
    ops.bind_attention("attn_draft_and_verify", _Unrun())
    graphs = []

    def layer(q, k, v, indptr, cache, idx, kvp, last):
        torch.ops.bsx.update_kv(k, v, indptr, cache, idx, kvp, last, 16)
        return torch.ops.bsx.attn_draft_and_verify(q, cache)

    f = torch.compile(layer, backend=_fake_backend(graphs), fullgraph=True)
    q = torch.zeros(10, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(10, 8, 128, dtype=torch.bfloat16)
    cache = torch.zeros(4, 2, 16, 8, 128, dtype=torch.bfloat16)
    out = f(q, k, k, _i32(0, 5, 10), cache, _i32(0, 1, 2, 3), _i32(0, 2, 4), _i32(3, 3))
    assert out.shape == q.shape and out.dtype == q.dtype
    assert len(graphs) == 1
    code = graphs[0].code
    assert "torch.ops.bsx.update_kv" in code and "torch.ops.bsx.attn_draft_and_verify" in code


def test_fused_update_and_attention_operator_traces():
    ops.bind_attention("attn_verify_fused", _Unrun())
    graphs = []
    f = torch.compile(lambda q, k, v, c: torch.ops.bsx.attn_verify_fused_with_append(q, k, v, c),
                      backend=_fake_backend(graphs), fullgraph=True)
    q = torch.zeros(10, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(10, 8, 128, dtype=torch.bfloat16)
    cache = torch.zeros(4, 2, 16, 8, 128, dtype=torch.bfloat16)
    out = f(q, k, k, cache)
    assert out.shape == q.shape and len(graphs) == 1


def test_acceptance_operators_trace_with_the_reference_dtypes():
    graphs = []
    be = _fake_backend(graphs)
    draft = torch.zeros(4, 4, dtype=torch.int64)
    logits = torch.zeros(4, 5, 100, dtype=torch.bfloat16)
    g = torch.compile(lambda d, x: torch.ops.bsx.evaluate_posterior_greedy(d, x, -1, 0),
                      backend=be, fullgraph=True)(draft, logits)
    assert [(tuple(t.shape), t.dtype) for t in g] == [((4, 1), torch.int64), ((4,), torch.int64),
                                                      ((4, 1), torch.bool)]
    s = torch.compile(lambda d, x, u: torch.ops.bsx.evaluate_posterior_sampling(
        d, x, -1, 0.6, 0.95, 20, u), backend=be, fullgraph=True)(draft, logits, torch.zeros(4, 5))
    assert [(tuple(t.shape), t.dtype) for t in s] == [((4, 1), torch.int32), ((4,), torch.int32),
                                                      ((4, 1), torch.bool)]
    assert len(graphs) == 2


def test_binding_rejects_bad_names_and_rebinds():
    with pytest.raises(ValueError):
        ops.bind_attention("not a name", _Unrun())
    a, b = _Unrun(), _Unrun()
    op1 = ops.bind_attention("attn_prefill", a)
    op2 = ops.bind_attention("attn_prefill", b)
    assert op1 is op2 and ops._WRAPPERS["attn_prefill"] is b


def test_operators_refuse_cpu_tensors():
    """The real implementations run the HIP library only: CPU tensors are refused."""
    k = torch.zeros(10, 8, 128, dtype=torch.bfloat16)
    cache = torch.zeros(4, 2, 16, 8, 128, dtype=torch.bfloat16)
    with pytest.raises((ValueError, RuntimeError)):
        torch.ops.bsx.update_kv(k, k, _i32(0, 5, 10), cache, _i32(0, 1, 2, 3), _i32(0, 2, 4),
                                _i32(3, 3), 16)
