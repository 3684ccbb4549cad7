"""Randomized verify-attention cases through the wrapper (plan + run, the FlashInfer call
at batchspec/models/modules/attention/standard.py:69 planned as in
batchspec/backends/standard_engine.py:130-143 and mtp_engine.py:420-432), each against the
fp32 oracle with the bounds of tests/attn_parity.py.  The cases mix bf16 and fp16, head
dims 64 and 128 with several GQA ratios, page sizes 1-64, ragged query lengths (0 included)
and contexts (0 included), and the four mask modes: causal, none, draft trees (per-token
ancestor words, up to 32 nodes) and the sink + window view."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd.workloads import make_verify_batch
from oracle import attention as OA
from tests import attn_parity as AP

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
N_CASES = 40
HEADS = [(64, 8, 2), (128, 32, 8), (128, 8, 8), (64, 16, 2), (128, 16, 4)]


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _case(rng):
    dtype = [torch.bfloat16, torch.float16][int(rng.integers(2))]
    D, Hq, Hkv = HEADS[int(rng.integers(len(HEADS)))]
    ps = int(rng.choice([1, 8, 16, 32, 64]))
    B = int(rng.integers(1, 13))
    mode = str(rng.choice(["causal", "causal", "none", "tree", "streaming"]))
    if mode == "tree":
        qo = rng.integers(1, 33, size=B)
    elif mode == "streaming":
        qo = rng.integers(0, 2, size=B)
    else:
        qo = rng.choice([0, 1, 2, 5, 8, 16, 40], size=B)
    ctx = rng.integers(0, 3001, size=B)
    ctx[rng.random(B) < 0.15] = 0
    scale = float(rng.choice([0.5, 1.0, 1.5]))
    sink, window = int(rng.choice([0, 4, 64])), int(rng.choice([32, 200, 512]))
    return dtype, D, Hq, Hkv, ps, B, mode, qo.astype(np.int64), ctx.astype(np.int64), scale, \
        sink, window


@pytest.mark.parametrize("case", range(N_CASES))
def test_random_attention_case(case):
    rng = np.random.default_rng(5000 + case)
    dtype, D, Hq, Hkv, ps, B, mode, qo, ctx, scale, sink, window = _case(rng)
    say(f"case {case}: {dtype} D={D} H={Hq}/{Hkv} ps={ps} B={B} mode={mode} qo={qo.tolist()} "
        f"ctx={ctx.tolist()} scale={scale}" + (f" sink={sink} window={window}"
                                               if mode == "streaming" else ""))
    b = make_verify_batch(B, 0, 0, 0, Hq, Hkv, D, ps, dtype=dtype, scale=scale, seed=7000 + case,
                          qo_lens=qo, ctx=ctx, tree_nodes=32 if mode == "tree" else 0).to(DEV)
    if int(qo.sum()) == 0:
        return  # nothing to attend
    ws = torch.empty(256 << 20, dtype=torch.uint8, device=DEV)
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    kw, okw = {}, {}
    if mode == "tree":
        kw["tree_mask_words"] = b.mask_words
    if mode == "streaming":
        kw.update(sink_tokens=sink, window_tokens=window)
        okw.update(sink=sink, window=window)
    w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, Hq, Hkv, D, ps,
           causal=mode in ("causal", "streaming"), q_data_type=dtype, **kw)
    out = w.run(b.q, b.cache)
    torch.cuda.synchronize()

    omode = {"causal": "causal", "none": "none", "streaming": "streaming", "tree": "custom"}[mode]
    if mode == "tree":
        # dense mask per request: every prefix column plus the ancestor block
        flat = []
        qi = b.qo_indptr.cpu().numpy()
        for r, L in enumerate(b.kv_lens):
            q_r = int(qi[r + 1] - qi[r])
            wr = b.mask_words[qi[r]: qi[r + 1]]
            blk = ((wr[:, None].astype(np.uint64) >> np.arange(q_r, dtype=np.uint64)) & 1)
            flat.append(np.concatenate([np.ones((q_r, L - q_r), bool), blk.astype(bool)],
                                       1).ravel())
        okw["custom_mask"] = np.concatenate(flat)
    ref = OA.verify_attention(b.q.float().cpu().numpy(), b.cache.float().cpu().numpy(),
                              b.qo_indptr.cpu().numpy(), b.kv_indptr.cpu().numpy(),
                              b.kv_indices.cpu().numpy(), b.kv_last_page_len.cpu().numpy(),
                              ps, mode=omode, **okw)
    AP.check(out, ref)
