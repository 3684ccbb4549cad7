"""Writes the golden fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

BatchSpec holds no golden tensors for its verify path (its one test, a checkpoint diff,
pins nothing here), so these vectors come from computations that are independent of
the oracle under test:
  config1_attention.npz  BASELINE config 1 inputs (B=4, ctx U[64,256], qo=5 causal, 8/2
                         heads, D=64, page 16, random page permutation, fp32 N(0,1)) and
                         the output / lse of torch float64 scaled_dot_product_attention
                         with an explicit bottom-right causal mask on the gathered pages
                         (batchspec/backends/standard_engine.py:132-143 plans causal=True).
  config1_append.npz     the same page table and cache: the 5 new K/V rows per request
                         and the (page, slot) each lands in, from a direct loop over the
                         positions of batchspec/models/modules/kv_cache.py:64-83 (every
                         other slot of the cache stays as it was).
  config1_greedy.npz     config 1 greedy acceptance over V=1000 (draft = target argmax
                         with probability 0.7): bonus / accept_nums / eos_accepted from
                         the reference's own tensor expressions (mtp_engine.py:553-560,747)
                         written in torch.
  chain_small.npz        chain speculative sampling, V=16, with the float64 sequential rule
                         (accept x_i iff u_i q_i(x_i) < p_i(x_i); residual / bonus draw by
                         inverse CDF); uniforms whose decisions lie within 1e-4 of a
                         boundary are redrawn, so the expected ids do not depend on rounding.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))


def config1_inputs():
    from batchspec_amd.workloads import config1
    b = config1(device="cpu", dtype=torch.float32)
    return b


def sdpa_reference(b):
    q = b.q.double()
    cache = b.cache.double()
    qo = b.qo_indptr.numpy()
    kvp = b.kv_indptr.numpy()
    idx = b.kv_indices.numpy()
    last = b.kv_last_page_len.numpy()
    ps = b.page_size
    Hq, Hkv, D = b.num_qo_heads, b.num_kv_heads, b.head_dim
    out = torch.zeros_like(q)
    lse = torch.full((q.shape[0], Hq), float("-inf"), dtype=torch.float64)
    for r in range(len(qo) - 1):
        npg = kvp[r + 1] - kvp[r]
        L = (npg - 1) * ps + last[r]
        pages = torch.from_numpy(idx[kvp[r]:kvp[r + 1]].astype(np.int64))
        kv = cache[pages]                        # [npg, 2, ps, Hkv, D]
        K = kv[:, 0].reshape(-1, Hkv, D)[:L]     # [L, Hkv, D]
        V = kv[:, 1].reshape(-1, Hkv, D)[:L]
        Q = q[qo[r]:qo[r + 1]]                   # [n, Hq, D]
        n = Q.shape[0]
        t = torch.arange(n)[:, None]
        j = torch.arange(L)[None, :]
        mask = j <= (L - n) + t                  # bottom-right causal
        g = Hq // Hkv
        Kx = K.repeat_interleave(g, dim=1).permute(1, 0, 2)   # [Hq, L, D]
        Vx = V.repeat_interleave(g, dim=1).permute(1, 0, 2)
        Qx = Q.permute(1, 0, 2)                               # [Hq, n, D]
        o = torch.nn.functional.scaled_dot_product_attention(Qx, Kx, Vx, attn_mask=mask)
        out[qo[r]:qo[r + 1]] = o.permute(1, 0, 2)
        s = (Qx @ Kx.transpose(1, 2)) / np.sqrt(D)
        s = s.masked_fill(~mask, float("-inf"))
        lse[qo[r]:qo[r + 1]] = torch.logsumexp(s, dim=-1).permute(1, 0)
    return out, lse


def write_attention(b):
    out, lse = sdpa_reference(b)
    np.savez_compressed(HERE / "config1_attention.npz", q=b.q.numpy(), cache=b.cache.numpy(),
                        qo_indptr=b.qo_indptr.numpy(), kv_indptr=b.kv_indptr.numpy(),
                        kv_indices=b.kv_indices.numpy(),
                        kv_last_page_len=b.kv_last_page_len.numpy(), page_size=b.page_size,
                        out=out.float().numpy(), lse=lse.float().numpy())


def write_append(b):
    qo = b.qo_indptr.numpy()
    kvp = b.kv_indptr.numpy()
    idx = b.kv_indices.numpy()
    last = b.kv_last_page_len.numpy()
    ps = b.page_size
    pages, slots = [], []
    for r in range(len(qo) - 1):
        seq_len = (kvp[r + 1] - kvp[r] - 1) * ps + last[r]
        n = qo[r + 1] - qo[r]
        for i in range(n):
            pos = seq_len - n + i
            pages.append(int(idx[kvp[r] + pos // ps]))
            slots.append(int(pos % ps))
    np.savez_compressed(HERE / "config1_append.npz", k_new=b.k_new.numpy(), v_new=b.v_new.numpy(),
                        target_page=np.array(pages, np.int32), target_slot=np.array(slots, np.int32))


def write_greedy():
    from batchspec_amd.workloads import greedy_case
    g = greedy_case(seed=1001)
    eos = 2
    # the reference's expressions (mtp_engine.py:747 argmax, :553-560 evaluation)
    preds = g.target_logits.argmax(-1)
    draft = g.draft_tokens
    k = draft.shape[1]
    flags = preds[:, :k] == draft
    accept = flags.sum(1) + 1
    bonus = preds.gather(1, (accept - 1)[:, None])
    eos_acc = ((draft == eos) & flags).any(1, keepdim=True)
    # a few eos drafts so the eos branch is exercised
    np.savez_compressed(HERE / "config1_greedy.npz", target_logits=g.target_logits.numpy(),
                        draft=draft.numpy(), eos=eos, bonus=bonus.numpy(), accept=accept.numpy(),
                        eos_accepted=eos_acc.numpy())


def chain_float64(q, p, draft, u, margin=1e-4):
    """Sequential chain rule in float64.  Returns ids [B, k+1] (-1 pad), accepted, emitted,
    or None for a row whose decision lies within `margin` of a boundary."""
    B, k, V = q.shape
    ids = np.full((B, k + 1), -1, np.int32)
    acc = np.zeros(B, np.int32)
    emi = np.zeros(B, np.int32)
    ok = np.ones(B, bool)
    for b in range(B):
        j = k
        for i in range(k):
            x = draft[b, i]
            lhs, rhs = u[b, i] * q[b, i, x], p[b, i, x]
            if abs(lhs - rhs) < margin:
                ok[b] = False
            if lhs < rhs:
                acc[b] += 1
            elif j == k:
                j = i
        emi[b] = j
        ids[b, :j] = draft[b, :j]
        w = np.maximum(p[b, j] - q[b, j], 0.0) if j < k else p[b, k]
        if w.sum() <= 0:
            w = p[b, j]
        c = np.cumsum(w) / w.sum()
        t = u[b, k]
        if np.min(np.abs(c - t)) < margin:
            ok[b] = False
        ids[b, j] = int(np.searchsorted(c, t, side="right"))
    return ids, acc, emi, ok


def write_chain():
    rng = np.random.default_rng(4242)
    B, k, V = 64, 3, 16
    tl = rng.normal(0, 1.5, (B, k + 1, V))
    dl = tl[:, :k] + rng.normal(0, 0.7, (B, k, V))
    p = np.exp(tl - tl.max(-1, keepdims=True)); p /= p.sum(-1, keepdims=True)
    q = np.exp(dl - dl.max(-1, keepdims=True)); q /= q.sum(-1, keepdims=True)
    p32, q32 = p.astype(np.float32), q.astype(np.float32)
    draft = np.stack([[rng.choice(V, p=q[b, i]) for i in range(k)] for b in range(B)]).astype(np.int64)
    u = rng.random((B, k + 1)).astype(np.float32)
    for _ in range(50):
        ids, acc, emi, ok = chain_float64(q32.astype(np.float64), p32.astype(np.float64), draft,
                                          u.astype(np.float64))
        if ok.all():
            break
        u[~ok] = rng.random((int((~ok).sum()), k + 1)).astype(np.float32)
    assert ok.all()
    np.savez_compressed(HERE / "chain_small.npz", draft_probs=q32, target_probs=p32, draft=draft,
                        uniforms=u, ids=ids, accepted=acc, emitted=emi)


if __name__ == "__main__":
    b = config1_inputs()
    write_attention(b)
    write_append(b)
    write_greedy()
    write_chain()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
