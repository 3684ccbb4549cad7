"""A torch.compile-d verify layer through the custom operators equals the eager layer.

BatchSpec compiles its forward (batchspec/backends/standard_engine.py:104-106,
batchspec/backends/mtp_engine.py:165-169) with attention and the KV update reached as
registered operators (batchspec/models/mtp_model.py:82-84,
batchspec/models/modules/attention/mtp.py:82-93, models/README.md:826-860).  Here a
per-layer forward (update_kv, then the bound attention operator) is compiled with
fullgraph=True by inductor and run at the config-2 shape; its output and the cache it
appends to must equal the eager layer's bit for bit, and the eager layer must match
the fp32 oracle.  The acceptance operators compiled the same way equal their eager
calls (greedy at [64, 5, 128256] bf16; sampling with the reference's defaults)."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd import ops
from batchspec_amd.workloads import config2, greedy_case
from tests import attn_parity as AP

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def layer(q, k, v, append_indptr, cache, kv_indices, kv_indptr, kv_last):
    torch.ops.bsx.update_kv(k, v, append_indptr, cache, kv_indices, kv_indptr, kv_last, 16)
    return torch.ops.bsx.attn_verify_compiled(q, cache)


def test_compiled_layer_equals_eager_at_config2():
    say("torch.compile(fullgraph=True) of update_kv + attention at config 2")
    b = config2(device=DEV)
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(
        torch.empty(256 << 20, dtype=torch.uint8, device=DEV), "NHD")
    w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, b.num_qo_heads,
           b.num_kv_heads, b.head_dim, b.page_size, causal=True, q_data_type=torch.bfloat16)
    ops.bind_attention("attn_verify_compiled", w)
    args = (b.qo_indptr, None, b.kv_indices, b.kv_indptr, b.kv_last_page_len)
    c_eager, c_comp = b.cache.clone(), b.cache.clone()
    ref = layer(b.q, b.k_new, b.v_new, args[0], c_eager, *args[2:])
    f = torch.compile(layer, fullgraph=True)
    got = f(b.q, b.k_new, b.v_new, args[0], c_comp, *args[2:])
    got2 = f(b.q, b.k_new, b.v_new, args[0], c_comp, *args[2:])  # the compiled code again
    torch.cuda.synchronize()
    assert torch.equal(c_comp, c_eager), "compiled update_kv wrote other cache contents"
    assert torch.equal(got, ref) and torch.equal(got2, ref), "compiled attention differs"
    b.cache = c_eager
    res = AP.oracle_per_request(b, "causal")[None]
    e, m = AP.check(ref, res[0])
    say(f"  compiled == eager bit for bit; eager vs oracle max err {e:.3g} (max|ref| {m:.3g})")


def test_compiled_acceptance_equals_eager():
    say("torch.compile(fullgraph=True) of the acceptance operators")
    g = greedy_case(B=64, k=4, V=128256, p_match=0.7, seed=2002, dtype=torch.bfloat16)
    x, d, u = g.target_logits.to(DEV), g.draft_tokens.to(DEV), g.uniforms.to(DEV)
    greedy = lambda d_, x_: torch.ops.bsx.evaluate_posterior_greedy(d_, x_, -1, 0)
    samp = lambda d_, x_, u_: torch.ops.bsx.evaluate_posterior_sampling(d_, x_, -1, 0.6, 0.95,
                                                                         20, u_)
    e_g = greedy(d, x)
    c_g = torch.compile(greedy, fullgraph=True)(d, x)
    e_s = samp(d, x, u)
    c_s = torch.compile(samp, fullgraph=True)(d, x, u)
    torch.cuda.synchronize()
    for a, b_ in zip(e_g + e_s, c_g + c_s):
        assert a.dtype == b_.dtype and torch.equal(a, b_)
    ref = bsx.evaluate_posterior(d, x, greedy=True, eos_token_id=-1)
    for a, b_ in zip(ref, e_g):
        assert torch.equal(a, b_)
    say(f"  greedy accept sum {int(e_g[1].sum())}, sampling accept sum {int(e_s[1].sum())}")
