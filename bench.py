"""Benchmark of the speculative-verification hot path on one MI355X.

Workload: Llama-3-8B shaped verify step of one decoder layer —
B=64 requests, context 1k-4k, k=4 chain draft (5 query tokens, causal), 32 query /
8 kv heads, head_dim 128, page size 16, random page permutation, bf16, values
N(0,1)*0.5 — i.e. the paged append of the 5 new K/V rows per request followed by
verify attention.  A "step" is append + attention over the whole batch; three
independent input sets rotate so the 256 MB last-level cache cannot serve repeats.

Printed: one JSON line with
  value       verify-attention HBM GB/s: algorithmic bytes of one attention pass
              (every K/V row of every request, Q, O and page ids once) / the mean
              duration of BatchPrefillWithPagedKVCacheWrapper.run(), hipEvent-timed
              on the stream the kernels run on (the pass is the attention kernel
              plus, for split requests, the merge of their partial results)
  roofline    the same pass against the 8 TB/s HBM peak; `traffic` is the HBM
              bytes per pass measured with rocprofv3 counters (profiles/)
  accepted_tok_s  accepted tokens/s of a 32-layer verify step: 32 x (append +
              attention) + fused greedy acceptance over [64, 5, 128256] bf16 logits
              (draft = target argmax with probability 0.7), reference acceptance rule
  stochastic_accept  config 5 (B=128, k=5, V=128256, bf16): time and HBM fraction
  cpu_baseline    the fp32 CPU oracle on a bounded sample of the same workload

`--extra-configs` adds verify attention at configs 4 (EAGLE trees), 3b (long context)
and 3a (sink+window draft view), the device tree masks of config 4, one step of the
sync-free page-table update at B=64 beside the host-synchronising torch mirror, and the
device-side attention schedule at config 2 with the attention pass run on it.

`--calibrate-copy` instead times a plain 1 GiB device copy (the known-size kernel
the HBM byte counters are scaled against).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "verify-attn HBM GB/s (% of 8 TB/s) + accepted tok/s, Llama-8B shape B=64 k=4"
TRAFFIC_FILE = ROOT / "profiles" / "verify_attn_config2_traffic.txt"


def attn_bytes(b) -> int:
    """Algorithmic bytes of one verify-attention pass: every K/V row of every request
    once, Q, O, page ids (and mask words) once."""
    import numpy as np
    kv_tokens = int(np.sum(b.kv_lens))
    nnz = b.q.shape[0]
    kv = kv_tokens * b.num_kv_heads * b.head_dim * 2 * 2
    qo = 2 * nnz * b.num_qo_heads * b.head_dim * 2
    pages = int(b.kv_indptr[-1].item()) * 4
    words = 0 if b.mask_words is None else nnz * 4
    return kv + qo + pages + words


def append_bytes(b) -> int:
    nnz = b.k_new.shape[0]
    return 2 * (2 * nnz * b.num_kv_heads * b.head_dim * 2)


def time_events(fn, iters: int, warmup: int):
    """Per-call durations (us) from hipEvents recorded on torch's current stream, which
    is the stream every batchspec_amd entry point launches on.  A GPU sleep is queued
    ahead of the timed calls so the host has enqueued them all before the first one
    runs: the events then bracket GPU time only, not the host's launch latency (which
    a graph-captured step, as BatchSpec runs it, does not pay per call either)."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    torch.cuda._sleep(50_000_000)
    for i in range(iters):
        starts[i].record()
        fn(i)
        ends[i].record()
    torch.cuda.synchronize()
    return [s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends)]


def median(xs):
    s = sorted(xs)
    return s[len(s) // 2]


def measured_traffic():
    """HBM bytes per attention pass from the committed rocprofv3 counter summary."""
    if not TRAFFIC_FILE.exists():
        return None
    m = re.search(r"^traffic_bytes_per_pass:\s*(\d+)", TRAFFIC_FILE.read_text(), re.M)
    return int(m.group(1)) if m else None


def extra_configs(dev, iters: int):
    """Verify attention at configs 4 (EAGLE tree), 3b (long context, split-KV) and 3a
    (the MagicDec draft over a 64-sink + 512-window view), each over rotating input sets
    (one for 3b: 6.4 GB of KV), timed like the headline pass."""
    import numpy as np
    import torch
    import batchspec_amd as bsx
    from batchspec_amd.workloads import config3, config4, make_verify_batch

    def run(name, sets, plan_kw, nbytes, n):
        ws = [torch.empty(512 << 20, dtype=torch.uint8, device=dev) for _ in sets]
        wr = []
        for b, w_buf in zip(sets, ws):
            w = bsx.BatchPrefillWithPagedKVCacheWrapper(w_buf, "NHD")
            kw = dict(plan_kw)
            if kw.pop("tree", False):
                kw["tree_mask_words"] = b.mask_words
            w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, b.num_qo_heads,
                   b.num_kv_heads, b.head_dim, b.page_size, q_data_type=torch.bfloat16, **kw)
            wr.append(w)
        outs = [torch.empty_like(b.q) for b in sets]
        k = len(sets)
        us = time_events(lambda i: wr[i % k].run(sets[i % k].q, sets[i % k].cache, out=outs[i % k]),
                         n, 3)
        t = sum(us) / len(us)
        nb = sum(nbytes) / k
        p = wr[0].plan_info
        return {"us": round(t, 2), "GB/s": round(nb / t / 1e3, 1),
                "frac": round(nb / t / 1e3 / HBM_PEAK_GBS, 4), "bytes": int(nb),
                "plan": {"workgroups": int(p.num_ctas), "segments": int(p.num_segments),
                         "split_requests": int(p.num_split_requests),
                         "shared_kv_tiles": int(p.shared_kv_tiles),
                         "heads_per_workgroup": int(p.heads_per_cta),
                         "waves_per_head": int(p.qblocks_per_cta)}}

    out = {}
    s4 = [config4(device=dev, seed=1004 + i) for i in range(3)]
    out["config4_tree_attention"] = run("4", s4, dict(causal=False, tree=True),
                                        [attn_bytes(b) for b in s4], iters)
    del s4
    s3 = [config3(device=dev, seed=1003)]
    out["config3b_verify_attention"] = run("3b", s3, dict(causal=True), [attn_bytes(s3[0])],
                                           max(5, iters // 3))
    del s3
    s3a = [make_verify_batch(32, 32768, 65536, 1, 32, 8, 128, 16, dtype=torch.bfloat16,
                             scale=0.5, seed=1003 + i, device=dev) for i in range(2)]

    def view_bytes(b):  # K/V rows of the 64 + 512 view, Q, O, page ids of the view
        view = int(np.sum(np.minimum(b.kv_lens, 576)))
        return (view * b.num_kv_heads * b.head_dim * 4 + 2 * b.q.numel() * 2
                + int(np.sum(np.minimum(np.diff(b.kv_indptr.cpu().numpy()), 36 + 1))) * 4)
    out["config3a_draft_attention"] = run("3a", s3a, dict(causal=True, sink_tokens=64,
                                                          window_tokens=512),
                                          [view_bytes(b) for b in s3a], iters)
    del s3a

    # Verify-step plumbing: the config-4 tree masks built on the device, and one step's
    # page-table update (insert the 25 MTP tokens, delete the rejected ones) at the
    # config-2 batch, against the host-synchronising torch mirror of the reference.
    import time
    from batchspec_amd.masks import tree_masks
    from batchspec_amd.page_table import DevicePageTable, PageTable
    from batchspec_amd.workloads import random_tree_parents
    rng = np.random.default_rng(1004)
    par = torch.from_numpy(np.stack([random_tree_parents(32, rng) for _ in range(32)])
                           .astype(np.int32)).to(dev)
    cl = torch.from_numpy(rng.integers(2048, 8192, 32).astype(np.int32)).to(dev)
    us = time_events(lambda i: tree_masks(par, cl), iters, 3)
    out["config4_tree_masks"] = {"us": round(sum(us) / len(us), 2), "requests": 32, "nodes": 32}
    acc = torch.from_numpy(rng.integers(1, 6, 64).astype(np.int32)).to(dev)
    rej = 25 - acc
    dpt = DevicePageTable(16, 64, 600, dev)
    dpt.insert_kv(torch.from_numpy(rng.integers(1024, 4096, 64).astype(np.int32)).to(dev))

    def step_dev(i):
        dpt.insert_kv(25)
        dpt.delete_kv(rej)
    us = time_events(step_dev, iters, 3)
    dpt.check()
    hpt = PageTable(16, 64, 600, dev)
    hpt.clear_kv()
    hpt.insert_kv(torch.from_numpy(rng.integers(1024, 4096, 64).astype(np.int32)).to(dev))
    for _ in range(3):
        hpt.insert_kv(25)
        hpt.delete_kv(rej)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        hpt.insert_kv(25)
        hpt.delete_kv(rej)
    torch.cuda.synchronize()
    host_us = (time.perf_counter() - t0) / iters * 1e6
    out["page_table_step"] = {"device_us": round(sum(us) / len(us), 2),
                              "torch_mirror_wall_us": round(host_us, 1), "requests": 64}

    # the device-side schedule at config 2 (one planner launch per step) and the
    # attention pass run on it; the host planner's wall time for comparison
    from batchspec_amd.workloads import config2
    s2 = [config2(device=dev, seed=1002 + i) for i in range(3)]
    ws2 = [bsx.BatchPrefillWithPagedKVCacheWrapper(torch.empty(256 << 20, dtype=torch.uint8,
                                                               device=dev), "NHD") for _ in s2]
    dev_args = [(b.qo_indptr.to(dev), b.kv_indptr.to(dev), b.kv_indices.to(dev),
                 b.kv_last_page_len.to(dev)) for b in s2]

    def plan_dev(i):
        b = s2[i % 3]
        ws2[i % 3].plan(*dev_args[i % 3], b.num_qo_heads, b.num_kv_heads, b.head_dim, b.page_size,
                        causal=True, q_data_type=torch.bfloat16, on_device=True, max_qo_len=5)
    plan_us = time_events(plan_dev, iters, 3)
    outs2 = [torch.empty_like(b.q) for b in s2]
    run_us = time_events(lambda i: ws2[i % 3].run(s2[i % 3].q, s2[i % 3].cache, out=outs2[i % 3]),
                         iters, 3)
    t = sum(run_us) / len(run_us)
    nb = sum(attn_bytes(b) for b in s2) / 3
    hw = bsx.BatchPrefillWithPagedKVCacheWrapper(torch.empty(256 << 20, dtype=torch.uint8,
                                                             device=dev), "NHD")
    t0 = time.perf_counter()
    for i in range(iters):
        b = s2[i % 3]
        hw.plan(dev_args[i % 3][0], dev_args[i % 3][1], dev_args[i % 3][2], dev_args[i % 3][3],
                b.num_qo_heads, b.num_kv_heads, b.head_dim, b.page_size, causal=True,
                q_data_type=torch.bfloat16)
    torch.cuda.synchronize()
    host_plan_us = (time.perf_counter() - t0) / iters * 1e6
    out["config2_device_plan"] = {"plan_kernel_us": round(sum(plan_us) / len(plan_us), 2),
                                  "attention_us": round(t, 2),
                                  "frac": round(nb / t / 1e3 / HBM_PEAK_GBS, 4),
                                  "host_plan_wall_us": round(host_plan_us, 1)}
    return out


def cpu_baseline(sets, budget_s: float = 12.0):
    """fp32 oracle (numpy paged gather + softmax attention) over the config-2 requests,
    cycling through the batch until about budget_s of CPU work; reported in the
    metric's unit (GB/s of the same algorithmic bytes)."""
    import numpy as np
    import torch
    from oracle import attention as OA
    try:
        from threadpoolctl import threadpool_info
        cores = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
    except Exception:
        cores = 1
    b = sets[0]
    q = b.q.float().cpu().numpy()
    qo = b.qo_indptr.cpu().numpy()
    kvp = b.kv_indptr.cpu().numpy()
    idx = b.kv_indices.cpu().numpy()
    last = b.kv_last_page_len.cpu().numpy()
    lens = b.kv_lens
    B = len(qo) - 1
    subs = []
    for r in range(B):
        pages = idx[kvp[r]:kvp[r + 1]]
        sub = b.cache[torch.from_numpy(pages.astype(np.int64)).to(b.cache.device)].float().cpu().numpy()
        subs.append((pages, sub))
    t_total, done_bytes, n_req = 0.0, 0, 0
    while t_total < budget_s:
        r = n_req % B
        pages, sub = subs[r]
        t0 = time.perf_counter()
        OA.verify_attention(q[qo[r]:qo[r + 1]], sub, [0, qo[r + 1] - qo[r]],
                            [0, len(pages)], np.arange(len(pages), dtype=np.int32),
                            last[r:r + 1], b.page_size, mode="causal")
        t_total += time.perf_counter() - t0
        done_bytes += (int(lens[r]) * b.num_kv_heads * b.head_dim * 2 * 2
                       + 2 * int(qo[r + 1] - qo[r]) * b.num_qo_heads * b.head_dim * 2
                       + len(pages) * 4)
        n_req += 1
    return {"value": round(done_bytes / t_total / 1e9, 3), "unit": "GB/s", "cores": int(cores),
            "kind": "port",
            "sample": f"{n_req} config-2 requests ({n_req / B:.1f} passes over the batch of {B}), "
                      f"fp32 numpy paged gather + softmax attention, {t_total:.1f} s of CPU time; "
                      "bytes counted as the bf16 algorithmic bytes of the GPU metric"}


def calibrate_copy(reps: int = 5) -> int:
    import torch
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    us = time_events(lambda i: dst.copy_(src), reps, 2)
    print(json.dumps({"calibration": "copy", "bytes_read": n, "bytes_written": n,
                      "us": round(sum(us) / len(us), 2),
                      "GB/s": round(2 * n / (sum(us) / len(us)) / 1e3, 1)}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-accept", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--extra-configs", action="store_true",
                    help="also time verify attention at configs 4, 3b and 3a")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); the "
              "verify path shards by request / kv head with no exchange, see the design notes.",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    if args.calibrate_copy:
        return calibrate_copy()

    import batchspec_amd as bsx
    from batchspec_amd.workloads import config2, greedy_case, stochastic_case

    dev = "cuda:0"
    torch.cuda.set_device(0)
    print("bench: building 3 config-2 input sets on the GPU", file=sys.stderr, flush=True)
    sets = [config2(device=dev, seed=1002 + i) for i in range(3)]
    ws = [torch.empty(256 << 20, dtype=torch.uint8, device=dev) for _ in sets]
    wrappers = []
    plan_us = []
    for b, w_buf in zip(sets, ws):
        w = bsx.BatchPrefillWithPagedKVCacheWrapper(w_buf, "NHD")
        t0 = time.perf_counter()
        w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, b.num_qo_heads,
               b.num_kv_heads, b.head_dim, b.page_size, causal=True, q_data_type=torch.bfloat16)
        plan_us.append((time.perf_counter() - t0) * 1e6)
        wrappers.append(w)
    outs = [torch.empty_like(b.q) for b in sets]
    abytes = [attn_bytes(b) for b in sets]
    pbytes = [append_bytes(b) for b in sets]

    def step(i):
        j = i % 3
        b = sets[j]
        bsx.append_kv(b.k_new, b.v_new, b.qo_indptr, b.cache, b.kv_indptr, b.kv_indices,
                      b.kv_last_page_len)
        wrappers[j].run(b.q, b.cache, out=outs[j])

    # --- timed steps (append + attention): barrier-free single GPU, synchronize on both
    # sides of exactly `steps` steps
    print(f"bench: {args.warmup} warmup + {args.steps} timed steps", file=sys.stderr, flush=True)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for i in range(args.steps):
        step(i)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = ev0.elapsed_time(ev1) / args.steps
    step_bytes = sum(abytes[i % 3] + pbytes[i % 3] for i in range(args.steps)) / args.steps

    # --- per-launch hipEvent timing of the attention pass and of the append
    attn_us = time_events(lambda i: wrappers[i % 3].run(sets[i % 3].q, sets[i % 3].cache,
                                                        out=outs[i % 3]), args.steps, 3)
    app_us = time_events(lambda i: bsx.append_kv(sets[i % 3].k_new, sets[i % 3].v_new,
                                                 sets[i % 3].qo_indptr, sets[i % 3].cache,
                                                 sets[i % 3].kv_indptr, sets[i % 3].kv_indices,
                                                 sets[i % 3].kv_last_page_len), args.steps, 3)
    t_attn = sum(attn_us) / len(attn_us)
    t_app = sum(app_us) / len(app_us)
    a_bytes = sum(abytes) / 3
    achieved = a_bytes / (t_attn * 1e-6) / 1e9
    p0 = wrappers[0].plan_info
    result = {
        "metric": METRIC,
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "config2: Llama-3-8B verify layer, B=64, ctx U[1024,4096], "
                               "k=4 (5 causal queries), 32/8 heads, D=128, page 16, random "
                               "page permutation, bf16; step = paged append + verify attention",
                   "batch": 64, "draft_len": 4, "num_qo_heads": 32, "num_kv_heads": 8,
                   "head_dim": 128, "page_size": 16},
        "pct_of_hbm_peak": round(100 * achieved / HBM_PEAK_GBS, 2),
        "step_gbs": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
        "attn_us": round(t_attn, 2),
        "attn_us_median": round(median(attn_us), 2),
        "append_us": round(t_app, 2),
        "append_GBs": round(sum(pbytes) / 3 / t_app / 1e3, 1),
        "attn_bytes": int(a_bytes),
        "plan_us": round(median(plan_us), 1),
        "plan": {"workgroups": int(p0.num_ctas), "segments": int(p0.num_segments),
                 "split_requests": int(p0.num_split_requests), "tiles": int(p0.total_tiles)},
        "wall_s": round(wall, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "kernel": "verify attention pass (verify_attn_kernel + merge_kernel)"},
    }

    if not args.skip_accept:
        # greedy acceptance at the config-2 shape: fused argmax over [64, 5, 128256] bf16
        g = greedy_case(B=64, k=4, V=128256, p_match=0.7, seed=2002, dtype=torch.bfloat16)
        gl, gd = g.target_logits.to(dev), g.draft_tokens.to(dev)
        acc_us = time_events(lambda i: bsx.evaluate_posterior(gd, gl, greedy=True, eos_token_id=-1),
                             args.steps, 3)
        _, acc_ref, _ = bsx.evaluate_posterior(gd, gl, greedy=True, eos_token_id=-1)
        _, acc_pre, _ = bsx.evaluate_posterior(gd, gl, greedy=True, eos_token_id=-1,
                                               accept_rule="prefix")
        t_acc = sum(acc_us) / len(acc_us)
        t_model = 32 * (t_attn + t_app) + t_acc
        n_ref, n_pre = int(acc_ref.sum()), int(acc_pre.sum())
        result["accepted_tok_s"] = round(n_ref / (t_model * 1e-6), 1)
        result["accepted_tok_s_prefix_rule"] = round(n_pre / (t_model * 1e-6), 1)
        result["mean_accept_len"] = {"reference_rule": n_ref / 64, "prefix_rule": n_pre / 64}
        gbytes = gl.numel() * 2
        result["greedy_accept"] = {"us": round(t_acc, 2), "GB/s": round(gbytes / t_acc / 1e3, 1),
                                   "frac": round(gbytes / t_acc / 1e3 / HBM_PEAK_GBS, 4)}
        result["verify_step_32_layers_us"] = round(t_model, 1)
        # accepted-KV compaction (collate_accepted_kv_cache) of the same accept counts over
        # three layers of config-2 shape (set 0's cache and two more of its shape; layers
        # share one page table): rows prev + i*(k+1) -> prev + i
        from batchspec_amd.collate import collate_accepted_kv_cache
        kvl = torch.from_numpy(np.ascontiguousarray(sets[0].kv_lens)).to(dev)
        prev = (kvl - 25).to(torch.int32)
        caches = [sets[0].cache] + [torch.empty_like(sets[0].cache) for _ in range(2)]
        col_us = time_events(lambda i: collate_accepted_kv_cache(
            acc_ref, prev, 4, caches, sets[0].kv_indptr, sets[0].kv_indices), args.steps, 3)
        t_col = sum(col_us) / len(col_us)
        moved = int((acc_ref.clamp(max=5) - 1).clamp(min=0).sum()) * 2 * 8 * 128 * 2 * 2 * 3
        result["collate_accepted_kv"] = {"us_3_layers": round(t_col, 2),
                                         "bytes_moved": moved,
                                         "GB/s": round(moved / t_col / 1e3, 1)}
        del gl, g, caches
        # stochastic acceptance (config 5)
        s = stochastic_case(device=dev)
        st_us = time_events(lambda i: bsx.sampling.chain_speculative_sampling_from_logits(
            s.draft_logits, s.draft_tokens, s.target_logits, 1.0, uniforms=s.uniforms),
            max(5, args.steps // 3), 2)
        t_st = sum(st_us) / len(st_us)
        sbytes = (s.target_logits.numel() + s.draft_logits.numel()) * 2
        result["stochastic_accept"] = {"us": round(t_st, 2), "GB/s": round(sbytes / t_st / 1e3, 1),
                                       "frac": round(sbytes / t_st / 1e3 / HBM_PEAK_GBS, 4),
                                       "bytes": sbytes}
        # the same acceptance with the reference's default filters (top_k=20, top_p=0.95)
        # applied to both distributions
        sf_us = time_events(lambda i: bsx.sampling.chain_speculative_sampling_from_logits(
            s.draft_logits, s.draft_tokens, s.target_logits, 1.0, uniforms=s.uniforms,
            top_k=20, top_p=0.95), max(5, args.steps // 3), 2)
        t_sf = sum(sf_us) / len(sf_us)
        result["stochastic_accept_top_k20_top_p095"] = {
            "us": round(t_sf, 2), "GB/s": round(sbytes / t_sf / 1e3, 1),
            "frac": round(sbytes / t_sf / 1e3 / HBM_PEAK_GBS, 4), "bytes": sbytes}
        del s

    if args.extra_configs:
        print("bench: configs 4, 3b, 3a", file=sys.stderr, flush=True)
        result.update(extra_configs(dev, args.steps))

    if not args.no_cpu_baseline:
        print("bench: CPU baseline (fp32 oracle, ~12 s)", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(sets)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
