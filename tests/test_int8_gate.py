"""The INT8 ALIGN gate follows the reference engine's rule
(xiaotu_moe/csrc/moe/moe_v2_packed4_w4a8.inc:409-433): forced by
XIAOTU_MOE_INT8_ALIGN=1, otherwise allowed by the format and T >=
XIAOTU_MOE_INT8_VNNI_MIN_TOKENS (default 160, <= 0 disables)."""
import pytest

from xtu_moe_amd.layer import INT8_FORCE_ENV, INT8_MIN_TOKENS_ENV, int8_align_on


@pytest.fixture(autouse=True)
def _clean_env(monkeypatch):
    monkeypatch.delenv(INT8_FORCE_ENV, raising=False)
    monkeypatch.delenv(INT8_MIN_TOKENS_ENV, raising=False)


def test_default_threshold_is_160():
    assert not int8_align_on(1)
    assert not int8_align_on(159)
    assert int8_align_on(160)
    assert int8_align_on(8192)


def test_not_allowed_by_format():
    assert not int8_align_on(8192, allowed=False)


def test_threshold_from_env(monkeypatch):
    monkeypatch.setenv(INT8_MIN_TOKENS_ENV, "4")
    assert int8_align_on(4) and not int8_align_on(3)
    monkeypatch.setenv(INT8_MIN_TOKENS_ENV, "0")
    assert not int8_align_on(8192)


def test_force_env_ignores_tokens_and_format(monkeypatch):
    monkeypatch.setenv(INT8_FORCE_ENV, "1")
    assert int8_align_on(1) and int8_align_on(1, allowed=False)
