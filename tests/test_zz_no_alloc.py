"""The batch drain that allocates nothing (ssla_hip_drain_batch_noalloc)
against the entry point it is a variant of: the batch-mode drain,
ssla_hip_drain_n_ex with opts.batch.  Both run the same kernel, so on the
same records, weights and initial state their results are equal bit for
bit: output slots, head rows, hidden state, tdrop counters and prediction
grid.  Two calls in a row, the second with fewer records (its scratch then
still holds the first call's rows), on three blocks.
"""
import ctypes

import numpy as np
import pytest

from ssla_hip import abi, events

pytestmark = pytest.mark.gpu

BATCH = 16


def say(*a):
    print("[gpu-case]", *a, flush=True)


def _noalloc(L, d, batch, sync=1):
    nb = d.cfg.n_blocks
    rings = (ctypes.c_void_p * nb)(*[b.ptr for b in d._rings])
    ns = (ctypes.c_int * nb)(*d._ns)
    outs = (ctypes.c_void_p * nb)(*[b.ptr for b in d._outs])
    heads = (ctypes.c_void_p * nb)(*[b.ptr for b in d._heads])
    return L.ssla_hip_drain_batch_noalloc(ctypes.byref(d.cfg), rings, ns, outs, heads, batch,
                                          None, sync)


def _state(d, b):
    return [d.hidden(b, li) for li in range(4)] + list(d.counters(b)) + list(d.preds(b))


def test_noalloc_batch_drain_equals_batch_drain(stub_dir):
    from ssla_hip import hybrid as H
    from ssla_hip import lib
    L = lib.load()
    nb = 3
    streams = [events.to_records(events.blob_records(2600, seed=60 + b)) for b in range(nb)]
    calls = [[s[:2000] for s in streams], [s[2000:2000 + 300 + 50 * b] for b, s in
                                           enumerate(streams)]]
    with H.Drain.from_weights_dir(stub_dir, n_blocks=nb) as ref, \
            H.Drain.from_weights_dir(stub_dir, n_blocks=nb) as na:
        for k, recs in enumerate(calls):
            say(f"call {k}: records per block {[r.size for r in recs]}, batch {BATCH}")
            ref.load_rings(recs, want_head=True)
            ref.run(batch=BATCH)
            r_out, r_head = ref.results()
            na.load_rings(recs, want_head=True)
            lib.check(_noalloc(L, na, BATCH), "drain_batch_noalloc")
            n_out, n_head = na.results()
            for b in range(nb):
                assert np.array_equal(n_out[b], r_out[b]), (k, b)
                assert np.array_equal(n_head[b], r_head[b]), (k, b)
                got, want = _state(na, b), _state(ref, b)
                assert all(np.array_equal(g, w) for g, w in zip(got, want)), (k, b)
            p3 = sum(int((o["pass3"] == 1).sum()) for o in n_out)
            say(f"call {k}: equal on all blocks ({p3} pass-3 records)")
        # arguments beyond the scratch's limits are refused before any launch
        for bad in (0, 33):
            assert _noalloc(L, na, bad) == abi.SSLA_ERR_ARG
            assert b"batch" in L.ssla_hip_last_error()
