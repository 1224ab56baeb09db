"""Host-side policy of the quant-method hook (no GPU): which layers stay in
HBM, when a host-resident layer streams through the ring, and when the INT8
ALIGN path is allowed -- each against the reference's own switches."""
import types

import pytest

from xtu_moe_amd import formats as F
from xtu_moe_amd import host_layer as HL
from xtu_moe_amd import layer as L


def test_layer_set_syntax():
    assert HL.parse_layer_set("0-4,10") == {0, 1, 2, 3, 4, 10}
    assert HL.parse_layer_set(" 7 , 2-3,x,5-") == {7, 2, 3}
    assert HL.parse_layer_set("") == set()


def test_layer_index_from_vllm_names():
    lay = lambda n: types.SimpleNamespace(layer_name=n)
    assert HL.layer_index(lay("model.layers.12.mlp.experts")) == 12
    assert HL.layer_index(lay("model.mtp.experts")) is None
    assert HL.layer_index(types.SimpleNamespace()) is None


def test_resident_list_wins(monkeypatch):
    monkeypatch.setenv(HL.RESIDENT_LAYERS_ENV, "0-2,5")
    lay = lambda n: types.SimpleNamespace(layer_name=f"model.layers.{n}.mlp.experts")
    assert HL.resident_decision(lay(1), 10 ** 15, "cuda:0", total=1)
    assert not HL.resident_decision(lay(3), 1, "cuda:0", total=10 ** 15)
    # unnamed layers are host-resident once a list is given (as the reference)
    assert not HL.resident_decision(types.SimpleNamespace(), 1, "cuda:0", total=10 ** 15)


def test_budget_fills_in_load_order(monkeypatch):
    monkeypatch.delenv(HL.RESIDENT_LAYERS_ENV, raising=False)
    monkeypatch.setenv(HL.HBM_FRACTION_ENV, "0.5")
    monkeypatch.setattr(HL, "_RESIDENT_BYTES", {})
    lay = types.SimpleNamespace(layer_name="model.layers.0.mlp.experts")
    got = [HL.resident_decision(lay, 30, "cuda:7", total=100) for _ in range(3)]
    assert got == [True, False, False]                # 30 fits 50, 60 does not
    assert HL.resident_decision(lay, 20, "cuda:7", total=100)   # 50 still fits
    assert HL._RESIDENT_BYTES == {"cuda:7": 50}
    monkeypatch.setenv(HL.HBM_FRACTION_ENV, "0")
    assert not HL.resident_decision(lay, 1, "cuda:6", total=100)


def test_prefill_threshold(monkeypatch):
    monkeypatch.delenv(HL.PREFILL_MIN_ENV, raising=False)
    assert HL.gpu_prefill_min_tokens() == HL.PREFILL_MIN_DEFAULT
    monkeypatch.setenv(HL.PREFILL_MIN_ENV, "0")      # the reference's "off"
    assert HL.gpu_prefill_min_tokens() == 0
    monkeypatch.setenv(HL.PREFILL_MIN_ENV, "4096")
    assert HL.gpu_prefill_min_tokens() == 4096


@pytest.mark.parametrize("env,want", [
    ({}, False), ({"XIAOTU_MOE_INT8": "1"}, True), ({"XIAOTU_MOE_INT8": "0"}, None),
    ({"XIAOTU_MOE_INT8": "0", "XIAOTU_MOE_INT8_ALIGN": "1"}, None),
    ({"XIAOTU_MOE_INT8_ALIGN": "1"}, False)])
def test_int8_dispatch_follows_the_reference_switches(monkeypatch, env, want):
    for k in ("XIAOTU_MOE_INT8", "XIAOTU_MOE_INT8_ALIGN", "XIAOTU_MOE_INT8_VNNI"):
        monkeypatch.delenv(k, raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    assert L.int8_dispatch(F.FMT_MXFP4) is want
    for fmt in (F.FMT_FP8, F.FMT_NVFP4, F.FMT_BF16):
        assert L.int8_dispatch(fmt) is False
    # forced at every size when ALIGN=1, else from the 160-token gate when allowed
    forced = env.get("XIAOTU_MOE_INT8_ALIGN") == "1"
    assert L.int8_align_on(1, bool(want)) == forced
    assert L.int8_align_on(160, bool(want)) == (forced or bool(want))


def test_int8_vnni_scheme_is_refused(monkeypatch):
    monkeypatch.delenv("XIAOTU_MOE_INT8_ALIGN", raising=False)
    monkeypatch.setenv("XIAOTU_MOE_INT8_VNNI", "1")
    with pytest.raises(NotImplementedError):
        L.int8_dispatch(F.FMT_MXFP4)
