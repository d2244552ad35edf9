"""MTP policy of generate() (engine/engine.py:105-118), host logic only (CPU)."""

import pytest

from qvex.engine import MTP_MODES, mtp_policy


def test_modes():
    head = object()
    assert MTP_MODES == ("off", "on", "auto")
    assert mtp_policy("on", head)() is True
    assert mtp_policy("off", head)() is False
    assert mtp_policy("auto", head)() is True        # no thermal governor on this device
    assert mtp_policy("auto", None)() is False       # no head loaded: plain decoding
    assert mtp_policy("off", None)() is False


def test_errors():
    with pytest.raises(ValueError):
        mtp_policy("on", None)                       # "MTP head not loaded", as the reference
    with pytest.raises(ValueError):
        mtp_policy("sometimes", object())
