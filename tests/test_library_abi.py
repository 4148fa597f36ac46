"""The C-ABI library loads on a machine without a GPU, exports every entry
point include/cq35.h declares, and its host-only entry points (configuration
validation and the weight ABI) agree with the CPU restatement. No device
work is issued here."""
import ctypes
import os
import re

import pytest

import cq35
import cq35.config as cc
from cq35 import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    import cq35._build as b
    if not os.path.exists(b.LIBRARY):
        b.build()
    return _lib.load()


def declared_functions():
    text = open(os.path.join(ROOT, "include", "cq35.h")).read()
    return sorted(set(re.findall(r"^(?:const )?\w+\*? ?\*?\s*(cq35_\w+)\(", text, re.M)))


def test_header_symbols_exported(lib):
    names = declared_functions()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.EXPORTED)
    assert lib.cq35_abi_version() == 2


@pytest.mark.parametrize("name", sorted(cc.PRESETS))
def test_presets_validate_and_weight_abi_matches(lib, oracle, name):
    cfg = cc.preset(name)
    c = cc.to_c(cfg)
    assert lib.cq35_config_validate(ctypes.byref(c)) == 0
    specs = oracle.weight_specs(cfg)
    assert cq35.weight_count(cfg) == len(specs)
    for i, (dtype, rows, cols, _kind) in enumerate(specs):
        info = cq35.weight_info(cfg, i)
        assert (info.dtype, info.rows, info.cols) == (0 if dtype == "bf16" else 1, rows, cols), i
        assert info.bytes == rows * cols * (2 if dtype == "bf16" else 4)


def test_invalid_configs_are_rejected(lib):
    base = cc.preset("tiny")
    for change, fragment in [
        (dict(kv_heads=3), "divisible"),
        (dict(rope_dim=128), "rotary"),
        (dict(full_interval=1), "both full and linear"),
        (dict(hidden=260), "multiples of 8"),
        (dict(experts=4), "dense model"),
    ]:
        cfg = dict(base, **change)
        c = cc.to_c(cfg)
        assert lib.cq35_config_validate(ctypes.byref(c)) == -1, change
        assert fragment in lib.cq35_last_error().decode(), (change, lib.cq35_last_error())
