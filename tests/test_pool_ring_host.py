"""Host logic of the resident pool and the ring stage (no GPU): the swap
policy on the reference's own known-answer cases
(scripts/test_expert_pool_policy.py), the XTUP pin table, local top-k
selection, staging tiles, and the fail-closed defaults."""
import ast
import inspect
import os
import struct
import types

import pytest
import torch

from xtu_moe_amd import expert_pool as EP
from xtu_moe_amd import ring as R
from xtu_moe_amd.expert_pool import LayerPool, plan_swap


# ------------------------------------------------------------------ plan_swap
def test_plan_swap_empty_or_quiet_does_nothing():
    assert plan_swap([], {1: 5}, 0) == ([], [])
    assert plan_swap([], {1: 5}, 4) == ([], [])
    assert plan_swap([0, 1], {}, 2) == ([], [])


def test_plan_swap_rate_limit_coldest_out_hottest_in():
    ev, ld = plan_swap([0, 1, 2, 3], {4: 100, 5: 90, 6: 80, 7: 70}, 4, hyst=0.0, maxswap=2)
    assert ev == [0, 1]
    assert sorted(ld) == [4, 5]


def test_plan_swap_hysteresis():
    assert plan_swap([0], {0: 100, 1: 110}, 1, hyst=0.25, maxswap=1) == ([], [])
    assert plan_swap([0], {0: 100, 1: 130}, 1, hyst=0.25, maxswap=1) == ([0], [1])


def test_plan_swap_default_rate_is_a_quarter_of_the_slots():
    ev, _ = plan_swap([0, 1, 2, 3], {4: 1, 5: 1, 6: 1, 7: 1}, 4, hyst=0.0, maxswap=0)
    assert len(ev) <= 1
    ev, _ = plan_swap(list(range(16)), {100 + i: 5 for i in range(16)}, 16, hyst=0.0)
    assert len(ev) == 4


def test_plan_swap_residents_never_in_the_wrong_list():
    ev, ld = plan_swap([0, 1, 2, 3], {0: 9, 1: 1, 4: 50}, 4, hyst=0.0, maxswap=4)
    assert 4 not in ev and 0 not in ld


def test_plan_swap_tie_direction():
    # equal (zero) counts: oldest slot first, or newest first with preserve_oldest
    assert plan_swap([7, 8, 9, 10], {20: 5}, 4, hyst=0.0, maxswap=1)[0] == [7]
    assert plan_swap([7, 8, 9, 10], {20: 5}, 4, hyst=0.0, maxswap=1, preserve_oldest=True)[0] == [10]


# ------------------------------------------------------------------ pin table
def test_pin_table_round_trip(tmp_path):
    table = {0: [5, 3, 9], 2: [1], 7: [250, 0]}
    p = tmp_path / "pin.bin"
    n = EP.write_pin_table(str(p), table, n_layers=8, n_experts=256)
    assert n == 6
    raw = p.read_bytes()
    assert len(raw) == 20 + 4 * n   # the header is 20 bytes, not 16
    assert raw[:4] == b"XTUP" and struct.unpack_from("<I", raw, 4)[0] == 1
    assert EP.load_pin_table(str(p)) == table


def test_pin_table_rejects_bad_magic_and_truncation(tmp_path):
    p = tmp_path / "bad.bin"
    p.write_bytes(struct.pack("<4sIIII", b"XTUQ", 1, 1, 8, 0))
    with pytest.raises(ValueError):
        EP.load_pin_table(str(p))
    p.write_bytes(struct.pack("<4sIIII", b"XTUP", 1, 1, 8, 3) + struct.pack("<HH", 0, 1))
    with pytest.raises(ValueError):
        EP.load_pin_table(str(p))


# ------------------------------------------------------------ local selection
def test_select_local_topk_keeps_table_order_and_cuts_after_mapping():
    assert EP.select_local_topk([9, 3, 7, 3, 1], None, 10, 3) == [9, 3, 7]
    # expert-parallel map: half the global ids belong to another rank; the cut
    # applies to local ids, so this rank still gets `cap` of them
    em = torch.tensor([-1, 0, -1, 1, -1, 2, -1, 3])
    assert EP.select_local_topk([0, 2, 1, 4, 3, 5, 7], em, 4, 3) == [0, 1, 2]
    assert EP.select_local_topk([0, 2, 4], em, 4, 2) == []
    assert EP.select_local_topk([5, 1, 5], None, 4, 0) == [1]


def test_build_layer_pool_off_by_default(monkeypatch):
    monkeypatch.delenv(EP.ENV_ON, raising=False)
    assert EP.build_layer_pool(None, "cpu", 256, 128, 32, 8, 0, None) is None
    monkeypatch.setenv(EP.ENV_ON, "1")
    monkeypatch.setenv(EP.ENV_TABLE, "/nonexistent/pin.bin")
    assert EP.build_layer_pool(None, "cpu", 256, 128, 32, 8, 0, None) is None


# ------------------------------------------------------- fail-closed defaults
def _stub(**kw):
    base = dict(nslots=0, _hits=None, _win_t=torch.zeros((), dtype=torch.int64))
    base.update(kw)
    return types.SimpleNamespace(**base)


def test_maybe_adapt_does_nothing_by_default(monkeypatch):
    monkeypatch.delenv(EP.ENV_WINDOW, raising=False)
    assert LayerPool.maybe_adapt(_stub()) == 0
    assert LayerPool.maybe_adapt(_stub(nslots=4)) == 0
    busy = _stub(nslots=4, _hits=object(), _win_t=torch.full((), 999, dtype=torch.int64))
    assert LayerPool.maybe_adapt(busy) == 0                         # staging may be active
    assert LayerPool.maybe_adapt(busy, staging_active=False) == 0   # no window configured


def _code(fn) -> str:
    """Executable source of a method: docstring and comments dropped."""
    src = inspect.getsource(fn)
    tree = ast.parse("\n".join(l[4:] if l.startswith("    ") else l for l in src.splitlines()))
    f = tree.body[0]
    body = f.body[1:] if isinstance(f.body[0], ast.Expr) and isinstance(f.body[0].value, ast.Constant) else f.body
    return "\n".join(ast.unparse(b) for b in body)


def test_swap_rules_in_code():
    so = _code(LayerPool.swap_out)
    assert not any(t in so for t in ("del ", ".resize", "empty_cache", "torch.empty"))
    si = _code(LayerPool.swap_in)
    assert 0 < si.find("wait_event") < si.find("self.slotmap[int(new_expert)] =")
    assert "staging_active: bool=True" in inspect.signature(LayerPool.maybe_adapt).__str__().replace(" ", "") \
        or inspect.signature(LayerPool.maybe_adapt).parameters["staging_active"].default is True


# ----------------------------------------------------------------- ring tiles
def test_staging_tiles(monkeypatch):
    monkeypatch.delenv("XTU_STAGE_TILE_E", raising=False)
    assert R.staging_tile_experts(256) == 48
    assert R.staging_tile_experts(1) == 1
    assert R.staging_tile_experts(20) == 19   # never the whole layer
    monkeypatch.setenv("XTU_STAGE_TILE_E", "16")
    assert R.staging_tile_experts(256) == 16
    assert R.stage_tiles(40) == [(0, 16), (16, 32), (32, 40)]
    monkeypatch.setenv("XTU_STAGE_TILE_E", "999")
    assert R.staging_tile_experts(256) == 48
    assert R.stage_tiles(0) == []


def test_staging_bytes_counts_the_ring():
    from xtu_moe_amd import formats as F
    H, I = 7168, 2048
    per = F.algorithmic_bytes(F.FMT_FP8, 2 * I, H) + F.algorithmic_bytes(F.FMT_FP8, H, I)
    b = R.staging_bytes(256, H, I, ns=4, fmt=F.FMT_FP8, tile_e=16)
    assert b == 4 * 16 * per


# ------------------------------------------------------- slot-plane weights
def test_slot_planes_size_what_is_derived_from_them():
    """A pool's layer view claims E routed + NS shared experts but its planes
    hold only the pool's slots: per-expert work derived from the planes (the
    step-major MXFP4 scales, the INT8 weights) must cover the slots only."""
    from xtu_moe_amd import formats as F
    from xtu_moe_amd.layer import ExpertWeights
    H, I, S = 512, 256, 6
    mk = lambda N, K: torch.zeros((S, N * F.row_bytes(F.FMT_MXFP4, K)), dtype=torch.uint8)
    sc = lambda N, K: torch.zeros((S, F.scale_bytes(F.FMT_MXFP4, N, K)), dtype=torch.uint8)
    W = ExpertWeights(F.FMT_MXFP4, H, I, 16, 1, mk(2 * I, H), sc(2 * I, H), mk(H, I), sc(H, I),
                      mutable=True)
    assert W.n_experts == 17 and W.n_slots == S
    with pytest.raises(ValueError):     # planes of different expert counts
        ExpertWeights(F.FMT_MXFP4, H, I, 16, 1, mk(2 * I, H), sc(2 * I, H)[:4], mk(H, I),
                      sc(H, I))
    src = inspect.getsource(ExpertWeights.mx_pair_scales) + inspect.getsource(
        ExpertWeights.int8_planes)
    assert "self.n_experts" not in src


def test_pitched_copy_refuses_bad_sizes_before_any_copy():
    """copy_hostbuf_to_device_2d returns 0 for zero or negative heights,
    widths and pitches and for spans past the host buffer, without queuing a
    copy (the reference's 0-on-error contract)."""
    from xtu_moe_amd import formats as F
    from xtu_moe_amd.host_store import HostExpertStore
    from xtu_moe_amd.layer import ExpertWeights
    H, I, E = 256, 128, 3
    g = torch.Generator().manual_seed(0)
    w13 = torch.randn((E, 2 * I, H), generator=g) * 0.02
    w2 = torch.randn((E, H, I), generator=g) * 0.02
    c13, s13 = F.quantize_mxfp4(w13)
    c2, s2 = F.quantize_mxfp4(w2)
    W = ExpertWeights.from_dense(F.FMT_MXFP4, c13, s13, c2, s2, device="cpu")
    st = HostExpertStore.from_weights(W, pin=False)
    c = st.w13_cbytes
    for h, wdt, dp, sp, off in ((-1, c, c, 2 * c, 0), (E, -c, c, 2 * c, 0), (E, c, -c, 2 * c, 0),
                                (E, c, c, -2 * c, 0), (0, c, c, 2 * c, 0), (E, 0, c, 2 * c, 0),
                                (E, c, c, 2 * c, -1), (E + 1, c, c, 2 * c, 0),
                                (E, 2 * c + 1, 4 * c, 2 * c, 0)):
        assert st.copy_hostbuf_to_device_2d(0, 0, off, 1 << 40, dp, sp, wdt, h) == 0
