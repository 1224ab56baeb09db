"""xtu_segment_noalloc (the segmentation with a static device workspace, for
callers that cannot allocate) against xtu_segment with a caller workspace,
through the C ABI: every output bit-exact, on two calls in a row (the second
with a smaller batch, so stale counts of the first would show), and the
host-side rejection of a shape whose workspace exceeds the static array."""
import numpy as np
import pytest
import torch

from helpers import random_routing
from xtu_moe_amd import _lib
from xtu_moe_amd.layer import _p, _stream

pytestmark = pytest.mark.gpu

FIELDS = ("sorted_pair", "sorted_tok", "sorted_wts", "inv", "seg_start", "active", "n_active",
          "tile_expert", "tile_row0", "n_tiles", "expert_tile_start")


def _outputs(T, K, E, NS, bm, dev):
    A = max(T * K + T * NS, 1)
    NB = E + NS + 1
    mt = int(_lib.call("xtu_segment_max_tiles", T, K, E, NS, bm))
    i32 = dict(dtype=torch.int32, device=dev)
    o = dict(sorted_pair=torch.full((A,), -7, **i32), sorted_tok=torch.full((A,), -7, **i32),
             sorted_wts=torch.full((A,), float("nan"), dtype=torch.float32, device=dev),
             inv=torch.full((A,), -7, **i32), seg_start=torch.full((NB + 1,), -7, **i32),
             active=torch.full((NB,), -7, **i32), n_active=torch.full((1,), -7, **i32),
             tile_expert=torch.full((mt,), -7, **i32), tile_row0=torch.full((mt,), -7, **i32),
             n_tiles=torch.full((1,), -7, **i32),
             expert_tile_start=torch.full((NB + 1,), -7, **i32))
    return o


def _segment(noalloc, ids, wts, E, NS, bm, drop_zero, dev):
    T, K = ids.shape
    o = _outputs(T, K, E, NS, bm, dev)
    ptrs = [_p(o[f]) for f in FIELDS]
    head = (_p(ids), _p(wts), 0, T, K, E, NS, int(drop_zero), bm)
    if noalloc:
        _lib.call("xtu_segment_noalloc", *head, *ptrs, _stream())
    else:
        ws = torch.empty(int(_lib.call("xtu_segment_workspace_bytes", T, K, E, NS)),
                         dtype=torch.uint8, device=dev)
        _lib.call("xtu_segment", *head, _p(ws), *ptrs, _stream())
    torch.cuda.synchronize()
    return {f: o[f].cpu().numpy() for f in FIELDS}


def _check(T, K, E, NS, bm, seed, dev):
    ids, wts = random_routing(T, K, E, seed=seed, invalid_frac=0.03, zero_frac=0.05)
    ti, tw = torch.from_numpy(ids).to(dev), torch.from_numpy(wts).to(dev)
    for drop_zero in (True, False):
        ref = _segment(False, ti, tw, E, NS, bm, drop_zero, dev)
        got = _segment(True, ti, tw, E, NS, bm, drop_zero, dev)
        for f in FIELDS:
            np.testing.assert_array_equal(got[f].view(np.uint32), ref[f].view(np.uint32),
                                          err_msg=f"{f} T={T} E={E} drop_zero={drop_zero}")


def test_noalloc_segment_equals_workspace_segment_twice():
    dev = torch.device("cuda")
    print("noalloc: T=8192 K=8 E=256 NS=1", flush=True)
    _check(8192, 8, 256, 1, 64, seed=1, dev=dev)      # 18 blocks x 258 buckets of counts
    print("noalloc: T=700 K=10 E=512 NS=1 (smaller, after the larger call)", flush=True)
    _check(700, 10, 512, 1, 128, seed=2, dev=dev)


def test_noalloc_segment_rejects_oversize_workspace():
    dev = torch.device("cuda")
    T, K, E, NS = (1 << 17) + 256, 16, 2047, 0    # 513 blocks x 2048 buckets > 4 MiB
    assert _lib.call("xtu_segment_workspace_bytes", T, K, E, NS) > (4 << 20)
    dummy = torch.zeros(16, dtype=torch.int32, device=dev)
    args = [_p(dummy), _p(dummy), 0, T, K, E, NS, 1, 128] + [_p(dummy)] * 11 + [_stream()]
    rc = _lib.load().xtu_segment_noalloc(*args)   # rejected on the host, before any launch
    assert rc == 1   # hipErrorInvalidValue
