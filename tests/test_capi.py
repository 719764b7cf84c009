"""The C ABI library loads without a GPU and exports every function include/pgr.h declares;
the ctypes binding declares exactly those; the product refuses to run without the library."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys

import pytest

import _pgr_native as nat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pgr.h")


def declared_functions() -> set[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(pgr_[a-z0-9_]+)\s*\(", text))


def test_header_declares_the_expected_surface():
    names = declared_functions()
    for required in ("pgr_attn_step", "pgr_attn_stats_step", "pgr_attn_accumulate_step", "pgr_attn_fold_fixed_step",
                     "pgr_attn_finalize", "pgr_pager_new", "pgr_pager_on_step", "pgr_kv_decode_layer",
                     "pgr_kv_apply_tiers", "pgr_kv_begin_step", "pgr_kv_end_step"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(nat.LIB_PATH)
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_cover_exactly_the_header():
    assert set(nat.SIGNATURES) == declared_functions()


def test_abi_version_and_error_string():
    lib = nat.load()
    assert lib.pgr_abi_version() == nat.ABI_VERSION
    # A host-side validation failure needs no GPU: bad shapes fail before any launch.
    rc = lib.pgr_attn_step(None, None, None, None, None, None, None, None, 1, 14, 4, 8, 64, 0, 0.125, 0.0, None, 0,
                           None)
    assert rc == nat.PGR_ERR_INVALID
    assert "multiple" in nat.last_error()
    rc = lib.pgr_attn_step(None, None, None, None, None, None, None, None, 1, 34, 2, 8, 64, 0, 0.125, 0.0, None, 0,
                           None)
    assert rc == nat.PGR_ERR_UNSUPPORTED and "16" in nat.last_error()


def test_status_codes_match_the_header():
    text = open(HEADER).read()
    codes = {name: int(val) for name, val in re.findall(r"#define (PGR_(?:OK|ERR_[A-Z]+)) \(?(-?\d+)\)?", text)}
    assert codes["PGR_OK"] == 0 and len(codes) == 9
    for name, val in codes.items():
        if name != "PGR_OK":
            assert getattr(nat, name) == val, name
    assert sorted(codes.values()) == list(range(-8, 1))


def test_state_init_validates_before_any_launch():
    lib = nat.load()
    assert lib.pgr_attn_state_init(None, None, None, 0, 64, None) == 0  # nothing to write
    assert lib.pgr_attn_state_init(None, None, None, 4, 64, None) == nat.PGR_ERR_INVALID
    assert "null" in nat.last_error()
    assert lib.pgr_attn_state_init(None, None, None, 4, 0, None) == nat.PGR_ERR_INVALID
    assert lib.pgr_attn_state_init(None, None, None, -1, 64, None) == nat.PGR_ERR_INVALID


def test_workspace_size_is_deterministic_and_positive():
    lib = nat.load()
    a = lib.pgr_attn_workspace_bytes(8, 14, 2, 2048, 64, nat.MODE_FOLD, 16)
    b = lib.pgr_attn_workspace_bytes(8, 14, 2, 2048, 64, nat.MODE_FOLD, 16)
    assert a == b > 0
    assert lib.pgr_attn_workspace_bytes(8, 14, 2, 2048, 64, nat.MODE_STATS, 16) < a
    assert lib.pgr_attn_workspace_bytes(1, 14, 2, 0, 64, nat.MODE_FOLD, 16) == 0


def test_missing_library_fails_loudly():
    code = (
        "import os, sys; os.environ['PGR_LIBRARY'] = '/nonexistent/libpgr.so'; "
        f"sys.path.insert(0, {os.path.join(ROOT, 'rust-llm-pager_amd')!r}); "
        "import pager\n"
        "try:\n    pager.PyPager(1, 1, 1)\nexcept ImportError as e:\n    print('ImportError', e)\n"
    )
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True)
    assert "ImportError" in res.stdout, res.stdout + res.stderr


def test_no_product_module_imports_the_oracle():
    pkg = os.path.join(ROOT, "rust-llm-pager_amd")
    offenders = []
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(dirpath, f)).read()
                if re.search(r"^\s*(from|import)\s+oracle\b", src, flags=re.M):
                    offenders.append(f)
    assert not offenders
