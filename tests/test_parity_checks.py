"""The full-size attention parity checks can fail (CPU, no GPU needed).

The GPU tests at the benchmark shapes compare the kernels with the oracle through
tests/attn_parity.py.  These tests show, on CPU-generated inputs of the same shapes and
with the same planted keys, that the check rejects the mistakes it is meant to catch: a
missing causal or tree mask, a dropped last kv tile, an all-zeros output and an
off-by-one edge of the sink + window view; and that it accepts the reference rounded to
bf16 (the output precision of the kernels)."""
import numpy as np
import pytest
import torch

from batchspec_amd.workloads import config2, config3, config4, make_verify_batch
from tests import attn_parity as AP


def _bf16(x):
    return torch.from_numpy(x).to(torch.bfloat16).float().numpy()


def test_config2_shape_planted_check_rejects_mask_tile_and_zero_errors():
    b = config2()
    AP.plant_keys(b, "causal", seed=1)
    res = AP.oracle_per_request(b, "causal", mutations=("nomask", "droplast"))
    ref = res[None]
    assert AP.mismatch(_bf16(ref[0]), ref[0], ref[1], ref[1]) is None
    AP.assert_discriminates(ref, [("no mask", *res["nomask"]), ("last tile dropped", *res["droplast"]),
                                  ("zeros", np.zeros_like(ref[0]), None)])


def test_config3_shape_plain_inputs_reject_zeros_through_the_normalised_bound():
    """Without planted keys, over 32k-64k tokens |O| ~ 0.01 sits under the 2e-2 absolute
    floor of the elementwise bound; the normalised bound still rejects all zeros."""
    b = config3(batch=2)
    ref = AP.oracle_per_request(b, "causal")[None]
    z = np.zeros_like(ref[0])
    assert (np.abs(z - ref[0]) <= AP.ATOL + AP.RTOL * np.abs(ref[0])).all()
    assert "max|ref|" in AP.mismatch(z, ref[0])


def test_config4_shape_planted_check_rejects_tree_and_tile_errors():
    b = config4(batch=6)
    AP.plant_keys(b, "tree", seed=2)
    res = AP.oracle_per_request(b, "tree", mutations=("nomask", "droplast"))
    ref = res[None]
    assert AP.mismatch(_bf16(ref[0]), ref[0], ref[1], ref[1]) is None
    AP.assert_discriminates(ref, [("no tree mask", *res["nomask"]),
                                  ("last tile dropped", *res["droplast"])])


@pytest.mark.parametrize("sink,window", [(63, 512), (64, 480), (64, 513)])
def test_streaming_view_planted_check_rejects_edge_errors(sink, window):
    b = make_verify_batch(4, 3000, 9000, 1, 32, 8, 128, 16, dtype=torch.bfloat16, scale=0.5,
                          seed=41)
    AP.plant_keys(b, "streaming", seed=3, sink=64, window=512)
    ref = AP.oracle_per_request(b, "streaming", sink=64, window=512)[None]
    assert AP.mismatch(_bf16(ref[0]), ref[0], ref[1], ref[1]) is None
    bad = AP.oracle_per_request(b, "streaming", sink=sink, window=window)[None]
    AP.assert_discriminates(ref, [(f"sink {sink} window {window}", *bad)])


def test_planted_rows_carry_most_of_their_weight():
    """A planted key takes about e/(e+1) of its row's weight; a hidden one none."""
    b = make_verify_batch(3, 500, 2000, 5, 32, 8, 128, 16, dtype=torch.bfloat16, scale=0.5, seed=9)
    tg = AP.plant_keys(b, "causal", seed=4)
    ref = AP.oracle_per_request(b, "causal")[None][0]
    qo = b.qo_indptr.numpy()
    lens = b.kv_lens
    for (r, h, row), p in list(tg.items())[:40]:
        t, j = divmod(row, 4)
        L = int(lens[r])
        page = int(b.kv_indices[b.kv_indptr[r] + p // 16])
        v = b.cache[page, 1, p % 16, h].float().numpy()
        o = ref[qo[r] + t, h * 4 + j]
        cos = float(o @ v / (np.linalg.norm(o) * np.linalg.norm(v)))
        visible = p <= L - 5 + t
        assert (cos > 0.8) if visible else (cos < 0.5), (r, h, row, p, cos)
