"""GPU parity at the head layouts and vocabularies of the models BatchSpec ships configs
for (batchspec/models/configs/registry.py:7-132; head_dim = dim // n_head unless given,
model_config.py:53-54), whole and split over tensor-parallel ranks the way
batchspec/backends/utils/tensor_parallel.py:563-565 divides the heads.  The attention
tolerance is the north star's 2e-2 abs/rel; acceptance outputs are bit-exact against
the CPU oracle."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd import sampling as S
from batchspec_amd.workloads import greedy_case, make_verify_batch, stochastic_case
from oracle import accept as OAc
from oracle import attention as OA

pytestmark = pytest.mark.gpu
ATOL = RTOL = 2e-2
DEV = "cuda:0"

# (model, q heads, kv heads, head_dim) per rank
LAYOUTS = [
    ("llama-2-7b", 32, 32, 128),
    ("llama-2-13b", 40, 40, 128),
    ("llama-2-70b / llama-3-70b", 64, 8, 128),
    ("llama-3.2-1b", 32, 8, 64),
    ("Qwen2.5-7b", 28, 4, 128),
    ("Qwen2.5-7b tp2", 14, 2, 128),
    ("Qwen2.5-7b tp4", 7, 1, 128),
    ("Qwen2.5-14b/32b", 40, 8, 128),
    ("Qwen3-0.6B/1.7B", 16, 8, 128),
    ("DeepSeek-R1-Distill-Qwen-1.5B", 12, 2, 128),
    ("68m", 12, 12, 64),
    ("tinyllama", 32, 4, 64),
]


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def check(got, ref):
    g = got.float().cpu().numpy()
    assert np.isfinite(g).all()
    err = np.abs(g - ref) - (ATOL + RTOL * np.abs(ref))
    assert err.max() <= 0, f"max excess {err.max():.4g}, max abs err {np.abs(g - ref).max():.4g}"


def run(b, causal, **kw):
    ws = torch.empty(128 << 20, dtype=torch.uint8, device=DEV)
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, b.num_qo_heads,
           b.num_kv_heads, b.head_dim, b.page_size, causal=causal, q_data_type=b.q.dtype, **kw)
    out = w.run(b.q, b.cache)
    torch.cuda.synchronize()
    return out


def oracle(b, mode, **kw):
    return OA.verify_attention(b.q.float().cpu().numpy(), b.cache.float().cpu().numpy(),
                               b.qo_indptr.cpu().numpy(), b.kv_indptr.cpu().numpy(),
                               b.kv_indices.cpu().numpy(), b.kv_last_page_len.cpu().numpy(),
                               b.page_size, mode=mode, **kw)


@pytest.mark.parametrize("i", range(len(LAYOUTS)))
def test_chain_verify_at_model_layout(i):
    name, hq, hkv, d = LAYOUTS[i]
    say(f"chain verify (k=4, causal) at {name}: H={hq}/{hkv} D={d}")
    b = make_verify_batch(4, 30, 1200, 5, hq, hkv, d, 16, dtype=torch.bfloat16, scale=0.5,
                          seed=500 + i).to(DEV)
    check(run(b, True), oracle(b, "causal"))


@pytest.mark.parametrize("i", [0, 4, 7, 9, 11])
def test_tree_verify_at_model_layout(i):
    name, hq, hkv, d = LAYOUTS[i]
    say(f"tree verify (16 nodes) at {name}: H={hq}/{hkv} D={d}")
    b = make_verify_batch(3, 40, 900, 16, hq, hkv, d, 16, dtype=torch.bfloat16, scale=0.5,
                          seed=600 + i, tree_nodes=16).to(DEV)
    out = run(b, False, tree_mask_words=b.mask_words)
    qo = np.diff(b.qo_indptr.cpu().numpy())
    flat = []
    for r, L in enumerate(b.kv_lens):
        w = b.mask_words[b.qo_indptr[r].item(): b.qo_indptr[r + 1].item()]
        blk = ((w[:, None].astype(np.uint64) >> np.arange(qo[r], dtype=np.uint64)) & 1).astype(bool)
        flat.append(np.concatenate([np.ones((qo[r], L - qo[r]), bool), blk], 1).ravel())
    check(out, oracle(b, "custom", custom_mask=np.concatenate(flat)))


@pytest.mark.parametrize("V", [151936, 152064, 32000])
def test_greedy_acceptance_at_model_vocab(V):
    say(f"greedy acceptance, fused argmax, V={V} (B=8, k=4, bf16)")
    c = greedy_case(B=8, k=4, V=V, seed=V, dtype=torch.bfloat16)
    bonus, acc, eos = bsx.evaluate_posterior(c.draft_tokens.to(DEV), c.target_logits.to(DEV),
                                             greedy=True, eos_token_id=3)
    preds = c.target_logits.float().numpy().argmax(-1)
    flags = preds[:, :4] == c.draft_tokens.numpy()
    want = flags.sum(1) + 1
    np.testing.assert_array_equal(acc.cpu().numpy(), want)
    np.testing.assert_array_equal(bonus[:, 0].cpu().numpy(), preds[np.arange(8), want - 1])


@pytest.mark.parametrize("V,top_k,top_p", [(151936, 0, 0.0), (152064, 20, 0.95), (32000, 20, 0.95)])
def test_chain_acceptance_at_model_vocab(V, top_k, top_p):
    say(f"stochastic acceptance at V={V} top_k={top_k} top_p={top_p} (B=6, k=4, bf16)")
    c = stochastic_case(B=6, k=4, V=V, seed=V % 1000)
    got = S.chain_speculative_sampling_from_logits(c.draft_logits.to(DEV), c.draft_tokens.to(DEV),
                                                   c.target_logits.to(DEV), 1.0,
                                                   uniforms=c.uniforms.to(DEV), top_k=top_k,
                                                   top_p=top_p)
    args = (c.draft_logits.float().numpy(), c.draft_tokens.numpy(),
            c.target_logits.float().numpy(), 1.0)
    if top_k or top_p:
        ref = OAc.chain_filtered(*args, top_k, top_p, c.uniforms.numpy())
    else:
        ref = OAc.chain_logits(*args, c.uniforms.numpy())
    for a, r in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), r)
