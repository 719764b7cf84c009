"""The snippets of INTEGRATION.md, as a maintainer would copy them: the C sequence compiles
against include/pgr.h with every warning an error (as C and as C++, where a stray void*
argument does not convert silently), and the ctypes binding block returns the same
workspace size as the repository's own binding. CPU only: nothing is launched."""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

import _pgr_native as nat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DOC = os.path.join(ROOT, "INTEGRATION.md")


def _blocks(lang):
    return re.findall(r"```" + lang + r"\n(.*?)```", open(DOC).read(), flags=re.S)


# Declarations the C sequence assumes (named in the paragraph before it).
C_PRELUDE = """
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#include "pgr.h"
void integration_sequence(void);
void integration_sequence(void) {
  pgr_kv_config_t cfg;
  memset(&cfg, 0, sizeof cfg);
  uint64_t vram = 41u << 24, ram = 1u << 30, recent = 8;
  int32_t rows = 1, L = 22, n_new = 4;
  int64_t capacity_tokens = 8448, n_prompt = 8192;
  const void *q = NULL, *k_new = NULL, *v_new = NULL;
  void* out = NULL;
  float* mass_accum = NULL;
  int64_t accum_stride = 512;
  float scale = 0.125f;
  void* stream = NULL;
  int32_t completed[1];
  int32_t n_completed = 0;
  int64_t counts[5], moves[512], moves_cap = 512, scores_cap = 512;
  double scores[512];
"""


@pytest.mark.parametrize("compiler,lang", [("gcc", "c"), ("g++", "c++")])
def test_c_sequence_compiles_against_the_header(tmp_path, compiler, lang):
    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not installed")
    (snippet,) = [b for b in _blocks("c") if "pgr_kv_end_step_place" in b]
    src = tmp_path / ("seq.c" if lang == "c" else "seq.cpp")
    src.write_text(C_PRELUDE + snippet + "}\n")
    std = "-std=c11" if lang == "c" else "-std=c++17"
    res = subprocess.run([compiler, std, "-Wall", "-Wextra", "-Werror", "-Wno-unused-variable",
                          "-Wno-unused-but-set-variable", "-I", os.path.join(ROOT, "include"), "-c", str(src), "-o",
                          str(tmp_path / "seq.o")], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr


def test_ctypes_binding_block_matches_the_repository_binding(monkeypatch):
    binding = next(b for b in _blocks("python") if "pgr_attn_workspace_bytes.restype" in b)
    monkeypatch.chdir(ROOT)
    env = {"B": 64, "Hq": 16, "Hkv": 8, "Tc": 1 << 20, "D": 128}
    exec(binding, env)
    want = nat.load().pgr_attn_workspace_bytes(64, 16, 8, 1 << 20, 128, nat.MODE_FOLD, 16)
    assert env["ws_bytes"] == want > 0
    assert env["lib"].pgr_attn_workspace_bytes.restype is __import__("ctypes").c_size_t
