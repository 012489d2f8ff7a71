"""Slot fills (the role of ExpertPool._read, engine_v3.py:255-290): every
component of every filled slot holds exactly its record's bytes at the
record's component offset (verify_pool.py:64-87), for device-resident
sources and for a pinned host store, into a pool of component arrays (copy
kernels, batches wider than one launch) and into a pool of whole records
(one copy-engine copy per record)."""
import numpy as np
import pytest
import torch

from moe_stream_amd import geometry as G
from moe_stream_amd import synth
from moe_stream_amd.pool import SlotPool

pytestmark = pytest.mark.gpu


def _check(pool, store_u8, recs, slots):
    for c in pool.geom.components:
        got = pool.views[c.name][torch.as_tensor(slots, device=pool.device, dtype=torch.long)]
        got = got.contiguous().view(torch.uint8).reshape(len(slots), -1)
        want = store_u8[torch.as_tensor(recs, device=store_u8.device, dtype=torch.long),
                        c.offset:c.offset + c.nbytes].to(pool.device)
        assert torch.equal(got, want), c.name


@pytest.mark.parametrize("layout", ["components", "records"])
@pytest.mark.parametrize("geom,n_records,n_slots,n_fill", [
    (G.QWEN3_30B_A3B, 400, 512, 347),      # three launches of the batched kernel
    (G.GPT_OSS_120B, 24, 40, 21),          # 12 components, 5760-byte biases
    (G.SMALL, 64, 64, 64),
])
def test_device_source_fills_are_exact(geom, n_records, n_slots, n_fill, layout):
    store = synth.make_store(geom, n_records, "cuda", 20260701)
    pool = SlotPool(geom, n_slots, "cuda", store=store, layout=layout)
    rng = np.random.default_rng(20260702)
    recs = rng.choice(n_records, n_fill, replace=False)
    slots = rng.permutation(n_slots)[:n_fill]
    pool.fill(recs, slots)
    torch.cuda.synchronize()
    _check(pool, store, recs, slots)
    # refill half of the slots with other records: the new bytes replace the old
    recs2 = rng.choice(n_records, n_fill // 2, replace=False)
    pool.fill(recs2, slots[:n_fill // 2])
    torch.cuda.synchronize()
    _check(pool, store, recs2, slots[:n_fill // 2])
    _check(pool, store, recs[n_fill // 2:], slots[n_fill // 2:])


@pytest.mark.parametrize("layout", ["components", "records"])
def test_pinned_host_source_fills_are_exact(layout):
    geom = G.QWEN3_30B_A3B
    host = synth.make_host_store(geom, 40, "cuda", 20260703)
    dev = synth.make_store(geom, 40, "cuda", 20260703)
    pool = SlotPool(geom, 48, "cuda", store=host, layout=layout)
    recs, slots = np.arange(40)[::-1].copy(), np.arange(3, 43)
    pool.fill(recs, slots)
    torch.cuda.synchronize()
    _check(pool, dev, recs, slots)
    host.close()
