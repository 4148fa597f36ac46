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
    assert lib.cq35_abi_version() == 3


def header_parameters(name):
    text = open(os.path.join(ROOT, "include", "cq35.h")).read()
    m = re.search(r"^(?:const )?\w+\*? ?\*?\s*" + name + r"\(([^)]*)\)", text, re.M)
    args = [a.strip() for a in m.group(1).split(",") if a.strip() and a.strip() != "void"]
    return len(args)


def test_rust_binding_matches_header():
    """The Rust FFI crate a maintainer adds to catena-models
    (catena-models_amd/rust/catena-cq35-sys) declares only entry points of
    include/cq35.h, each with the header's parameter count, and the same
    constants."""
    src = open(os.path.join(ROOT, "catena-models_amd", "rust", "catena-cq35-sys", "src", "lib.rs")).read()
    decls = re.findall(r"pub fn (cq35_\w+)\(([^)]*)\)", src)
    assert len(decls) >= 20
    declared = set(declared_functions())
    for name, params in decls:
        assert name in declared, name
        n = len([p for p in params.split(",") if p.strip()])
        assert n == header_parameters(name), name
    header = open(os.path.join(ROOT, "include", "cq35.h")).read()
    for const in ["CQ35_ABI_VERSION", "CQ35_MATRIX_PROJECTIONS", "CQ35_MATRIX_EXPERTS", "CQ35_MATRIX_ATTENTION",
                  "CQ35_SPLIT_KEYS_DEFAULT"]:
        hv = re.search(r"#define " + const + r" (\d+)", header).group(1)
        rv = re.search(r"pub const " + const + r": \w+ = (\d+);", src).group(1)
        assert hv == rv, const
    # memory safety of the owning wrappers: a session borrows its model (the
    # model cannot be freed under a live session), the model is not shared
    # between threads, and host buffers are checked against the vocabulary
    # before the library writes to them
    assert re.search(r"pub struct Session<'m>\s*\{[^}]*_model: PhantomData<&'m Model>", src)
    assert re.search(r"pub fn session\(&self, capacity: i64\) -> anyhow::Result<Session<'_>>", src)
    assert "unsafe impl Sync for Model" not in src
    step = src.split("pub fn step(&mut self")[1].split("cq35_step(")[0]
    assert "l.len() >= self.vocab" in step
    batch = src.split("pub fn step_batch(")[1].split("cq35_step_batch(")[0]
    assert "l.len() >= need" in batch
    # the struct's fields in the header's order
    hfields = re.findall(r"^\s+(?:int32_t|float) (\w+);", header.split("typedef struct cq35_config")[1].split("}")[0], re.M)
    rfields = re.findall(r"pub (\w+): (?:i32|f32),", src.split("pub struct cq35_config")[1].split("}")[0])
    assert hfields == rfields


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
