"""CPU checks of the C-ABI boundary: the library loads, exports every entry
point include/helios_attn.h declares, and its host-only paths (argument
checks, workspace sizing) behave.  No kernel is launched."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch  # noqa: F401  (loads torch's HIP runtime before the library)

from helios_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "helios_attn.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]*?\b(hpa_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libheliosattn.so is not built; run python -m helios_amd.build")
    return _lib.load_library()


def test_header_declares_the_expected_entry_points():
    assert _declared() == sorted([
        "hpa_version", "hpa_last_error", "hpa_decode_workspace_size", "hpa_paged_decode",
        "hpa_paged_decode_noalloc", "hpa_paged_prefill", "hpa_kv_write", "hpa_kv_write_rope",
        "hpa_kv_gather", "hpa_copy_blocks", "hpa_step_tables",
    ])


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), f"{name} declared in helios_attn.h but not exported"
    assert set(_declared()) == set(_lib.SIGNATURES)


def test_version_matches_header(lib):
    m = re.search(r"#define HPA_VERSION (\d+)", HEADER.read_text())
    assert lib.hpa_version() == int(m.group(1))


def test_status_codes_match_header():
    text = HEADER.read_text()
    for name in ("HPA_OK", "HPA_ERR_ARG", "HPA_ERR_UNSUPPORTED", "HPA_ERR_WORKSPACE",
                 "HPA_ERR_LAUNCH", "HPA_F32", "HPA_F16", "HPA_BF16", "HPA_I8"):
        m = re.search(rf"#define {name} (\d+)", text)
        assert int(m.group(1)) == getattr(_lib, name), name


def test_noalloc_scratch_size_matches_header():
    m = re.search(r"#define HPA_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", HEADER.read_text())
    assert int(m.group(1)) << int(m.group(2)) == _lib.HPA_NOALLOC_SCRATCH_BYTES


def _ws(waves, rows, D, units):
    # a fixed 1 MiB region of int32 arrival counters (2^18 sequence x KV-head
    # units), then per wave two partial slots of rows x (m, l) floats and two
    # of rows x max(D, 16) floats of O
    if waves <= 1:
        return 0
    assert units <= 1 << 18
    return (1 << 20) + waves * (2 * rows * 2 * 4 + 2 * rows * max(D, 16) * 4)


def _waves(seqs, kv_heads, max_ctx, part_tokens):
    # host bound on the work, in 32-key steps plus 4 per (sequence, KV head)
    # unit, cut into slices of at least part_tokens / 32 steps, capped at 4096
    min_steps = max(1, ((part_tokens or 256) + 31) // 32)
    ub = seqs * kv_heads * (max(1, (max_ctx + 31) // 32) + 4)
    return max(1, min((ub + min_steps - 1) // min_steps, 4096))


def test_workspace_size(lib):
    # one unit that fits one slice: a single wave, every unit whole, no workspace
    assert _waves(1, 1, 32, 256) == 1
    assert lib.hpa_decode_workspace_size(1, 1, 4, 1, 64, 32, 256) == 0
    # two units of 8 steps (+4 each) over 8-step slices: rows = 14 / 2
    assert lib.hpa_decode_workspace_size(1, 1, 14, 2, 64, 256, 256) == _ws(_waves(1, 2, 256, 256), 7, 64, 2)
    # config 5 at the largest context: the 4096-wave cap, rows = 4 x 3
    assert _waves(256, 8, 32768, 0) == 4096
    assert lib.hpa_decode_workspace_size(256, 3, 32, 8, 128, 32768, 0) == _ws(4096, 12, 128, 2048)
    assert lib.hpa_decode_workspace_size(64, 1, 14, 2, 64, 4096, 32) == _ws(4096, 7, 64, 128)
    # config 5 at the wave cap fits the no-alloc entry's static scratch
    assert lib.hpa_decode_workspace_size(256, 3, 32, 8, 128, 32768, 0) <= _lib.HPA_NOALLOC_SCRATCH_BYTES


def test_argument_errors_return_status_without_a_gpu(lib):
    st = lib.hpa_paged_decode(None, None, 0, None, None, 0, None, None, 0, None, 1, None, 1, 1,
                              1, 1, 64, 16, 1, 16, 1.0, 0, None, 0, None)
    assert st == _lib.HPA_ERR_ARG
    assert b"null pointer" in lib.hpa_last_error()
    dummy = ctypes.c_void_p(16)
    st = lib.hpa_paged_decode(dummy, dummy, 1, dummy, dummy, 1, None, None, 0, dummy, 1, dummy,
                              1, 1, 4, 2, 64, 12, 8, 16, 1.0, 0, None, 0, None)
    assert st == _lib.HPA_ERR_UNSUPPORTED and b"block_size 12" in lib.hpa_last_error()
    st = lib.hpa_paged_decode(dummy, dummy, 1, dummy, dummy, 1, None, None, 0, dummy, 1, dummy,
                              1, 1, 4, 2, 48, 16, 8, 16, 1.0, 0, None, 0, None)
    assert st == _lib.HPA_ERR_UNSUPPORTED and b"head_dim 48" in lib.hpa_last_error()
    # more than 64 rows per KV head go to the prefill kernels, which refuse
    # head_dim 48 before launching anything
    st = lib.hpa_paged_decode(dummy, dummy, 1, dummy, dummy, 1, None, None, 0, dummy, 1, dummy,
                              1, 9, 8, 1, 48, 16, 8, 16, 1.0, 0, None, 0, None)
    assert st == _lib.HPA_ERR_UNSUPPORTED and b"head_dim 48" in lib.hpa_last_error()
    assert lib.hpa_decode_workspace_size(4, 9, 8, 1, 64, 4096, 0) == 0
    # int8 without scales
    st = lib.hpa_kv_write(dummy, dummy, 1, dummy, dummy, 3, None, None, 1, dummy, 1, dummy, dummy,
                          1, 1, 2, 64, 16, 8, None)
    assert st == _lib.HPA_ERR_ARG
    # rotary write: missing sin table, odd head_dim
    st = lib.hpa_kv_write_rope(dummy, dummy, 1, dummy, dummy, 1, None, None, 0, dummy, 1, dummy, dummy,
                               1, 1, 2, 64, 16, 8, dummy, None, 16, None)
    assert st == _lib.HPA_ERR_ARG and b"rotary" in lib.hpa_last_error()
    st = lib.hpa_kv_write_rope(dummy, dummy, 1, dummy, dummy, 1, None, None, 0, dummy, 1, dummy, dummy,
                               1, 1, 2, 63, 16, 8, dummy, dummy, 16, None)
    assert st == _lib.HPA_ERR_ARG and b"even head_dim" in lib.hpa_last_error()
    # step tables: wider than the resident rows, null resident array
    st = lib.hpa_step_tables(dummy, 1, None, 0, dummy, 4, 8, dummy, 9, None)
    assert st == _lib.HPA_ERR_ARG and b"step width 9" in lib.hpa_last_error()
    st = lib.hpa_step_tables(dummy, 1, None, 0, None, 4, 8, dummy, 8, None)
    assert st == _lib.HPA_ERR_ARG and b"null pointer" in lib.hpa_last_error()
    assert lib.hpa_step_tables(None, 0, None, 0, None, 0, 0, None, 0, None) == _lib.HPA_OK
    # empty batches are no-ops
    assert lib.hpa_paged_prefill(None, None, 0, None, None, 0, None, None, 0, None, 1, None, None,
                                 None, 0, 0, 0, 1, 1, 64, 16, 1, 1.0, None) == _lib.HPA_OK
    st = lib.hpa_paged_prefill(dummy, dummy, 1, dummy, dummy, 1, None, None, 0, dummy, 1, dummy, dummy,
                               dummy, 2, 4, -1, 8, 2, 64, 16, 8, 1.0, None)
    assert st == _lib.HPA_ERR_ARG and b"tokens -1" in lib.hpa_last_error()
