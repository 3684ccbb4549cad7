"""The allocation-free greedy acceptance (bsx_accept_greedy_noalloc, called through the
C ABI) against bsx_accept_greedy with a caller workspace: bit-identical bonus, accept and
eos outputs on consecutive calls whose second one is smaller, for fused-argmax logits
and for target ids; shapes beyond the scratch are refused."""
import ctypes
import sys

import numpy as np
import pytest
import torch

from batchspec_amd import _lib
from batchspec_amd.workloads import greedy_case
from oracle import accept as OAc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _call(lib, noalloc, draft, ids, logits, B, k, V, eos, mode):
    bonus = torch.full((B,), -7, dtype=torch.int64, device=DEV)
    acc = torch.full((B,), -7, dtype=torch.int64, device=DEV)
    eacc = torch.full((B,), 9, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    dt = 0 if logits is None else {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16,
                                   torch.float32: _lib.DTYPE_FP32}[logits.dtype]
    lp = None if logits is None else logits.data_ptr()
    ip = None if ids is None else ids.data_ptr()
    if noalloc:
        rc = lib.bsx_accept_greedy_noalloc(draft.data_ptr(), ip, lp, dt, B, k, V, eos, mode,
                                           bonus.data_ptr(), acc.data_ptr(), eacc.data_ptr(),
                                           stream)
    else:
        nbytes = int(lib.bsx_accept_greedy_ws_bytes(B, k, V))
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=DEV)
        rc = lib.bsx_accept_greedy(draft.data_ptr(), ip, lp, dt, B, k, V, eos, mode,
                                   bonus.data_ptr(), acc.data_ptr(), eacc.data_ptr(),
                                   ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "greedy")
    torch.cuda.synchronize()
    return bonus.cpu().numpy(), acc.cpu().numpy(), eacc.cpu().numpy()


@pytest.mark.parametrize("mode", [0, 1])
def test_noalloc_greedy_matches_the_workspace_entry_point(mode):
    lib = _lib.load()
    cases = [(64, 4, 128256, torch.bfloat16, 11), (8, 3, 32000, torch.float16, 12),
             (5, 2, 1000, torch.float32, 13)]
    for B, k, V, dt, seed in cases:  # each call smaller than the one before
        say(f"no-alloc greedy: B={B} k={k} V={V} {dt} mode={mode}")
        c = greedy_case(B=B, k=k, V=V, seed=seed, dtype=dt)
        draft = c.draft_tokens.to(DEV).contiguous()
        logits = c.target_logits.to(DEV).contiguous()
        eos = int(c.draft_tokens[0, 0])
        got = _call(lib, True, draft, None, logits, B, k, V, eos, mode)
        want = _call(lib, False, draft, None, logits, B, k, V, eos, mode)
        for g, w in zip(got, want):
            np.testing.assert_array_equal(g, w)
        ref = OAc.greedy_posterior(c.draft_tokens.numpy(), c.target_logits.float().numpy(), eos,
                                   "reference" if mode == 0 else "prefix")
        np.testing.assert_array_equal(got[0], ref[0][:, 0])
        np.testing.assert_array_equal(got[1], ref[1])
        ids = torch.from_numpy(OAc.argmax(c.target_logits.float().numpy())).to(DEV).contiguous()
        got_i = _call(lib, True, draft, ids, None, B, k, V, eos, mode)
        for g, w in zip(got_i, want):
            np.testing.assert_array_equal(g, w)


def test_noalloc_greedy_refuses_shapes_beyond_its_scratch():
    lib = _lib.load()
    B, k, V = 40000, 4, 128256  # 200000 rows of partials > BSX_NOALLOC_SCRATCH_BYTES
    assert lib.bsx_accept_greedy_ws_bytes(B, k, V) > _lib.NOALLOC_SCRATCH_BYTES
    p = ctypes.c_void_p(16)
    rc = lib.bsx_accept_greedy_noalloc(p, None, p, _lib.DTYPE_BF16, B, k, V, -1, 0, p, p, p, None)
    assert rc == _lib.BSX_ERR_CAPACITY
    assert b"allocation-free scratch" in lib.bsx_last_error()


_CAPTURE_SCRIPT = r'''
import sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from batchspec_amd import _lib
from batchspec_amd.workloads import greedy_case
DEV = "cuda:0"
lib = _lib.load()
B, k, V = 64, 4, 128256
c = greedy_case(B=B, k=k, V=V, seed=21, dtype=torch.bfloat16)
draft = c.draft_tokens.to(DEV).contiguous()
logits = c.target_logits.to(DEV).contiguous()
outs = [torch.full((B,), -7, dtype=torch.int64, device=DEV) for _ in range(2)]
eacc = torch.full((B,), 9, dtype=torch.uint8, device=DEV)

def call(stream):
    return lib.bsx_accept_greedy_noalloc(draft.data_ptr(), None, logits.data_ptr(),
                                         _lib.DTYPE_BF16, B, k, V, -1, 0, outs[0].data_ptr(),
                                         outs[1].data_ptr(), eacc.data_ptr(), stream)

# the first call of the entry point in this process happens during the capture (its
# per-device scratch address is looked up then)
g = torch.cuda.CUDAGraph()
s = torch.cuda.Stream()
with torch.cuda.stream(s):
    with torch.cuda.graph(g, stream=s):
        rc = call(s.cuda_stream)
assert rc == 0, lib.bsx_last_error()
ws = torch.empty(int(lib.bsx_accept_greedy_ws_bytes(B, k, V)), dtype=torch.uint8, device=DEV)
ref = [torch.empty(B, dtype=torch.int64, device=DEV) for _ in range(2)]
ref_e = torch.empty(B, dtype=torch.uint8, device=DEV)
st = torch.cuda.current_stream().cuda_stream
_lib.check(lib.bsx_accept_greedy(draft.data_ptr(), None, logits.data_ptr(), _lib.DTYPE_BF16,
                                 B, k, V, -1, 0, ref[0].data_ptr(), ref[1].data_ptr(),
                                 ref_e.data_ptr(), ws.data_ptr(), ws.numel(), st), "greedy")
torch.cuda.synchronize()
for rep in range(4):
    for t in outs:
        t.fill_(-7)
    eacc.fill_(9)
    logits.mul_(1.0)  # eager work on the same stream between replays
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(outs[0], ref[0]) and torch.equal(outs[1], ref[1]), rep
    assert torch.equal(eacc, ref_e), rep
print("capture ok", int(outs[1].sum()))
'''


def test_noalloc_greedy_captured_on_its_first_call():
    """A fresh process whose first call of bsx_accept_greedy_noalloc is made while a
    graph is being captured (the scratch address lookup included); four replays, with
    eager work between them, each equal to bsx_accept_greedy with a workspace."""
    import os
    import subprocess
    say("no-alloc greedy captured in a graph on its first call (fresh process)")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, root], capture_output=True,
                       text=True, timeout=300)
    say(r.stdout.strip()[-400:])
    assert r.returncode == 0, r.stderr[-2000:]
    assert "capture ok" in r.stdout
