"""The C-ABI library (CPU only, no kernel launches): it loads, exports every function include/sd_attn.h
declares, reports its ABI version, sizes workspaces, and rejects bad arguments with a status code and a
message before touching the GPU."""
import ctypes
import os
import re

import pytest

from nanovllm_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sd_attn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\**\s+\**(sd_[a-z_0-9]+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) == 24, names
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, name
    assert set(_lib.SIGNATURES) == set(names)


def test_abi_version(lib):
    version = int(re.search(r"#define SD_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert lib.sd_abi_version() == version


def test_workspace_sizes(lib):
    # 64 sequences x 8 kv heads = 512 (item, head) pairs fill the GPU with 8-wave workgroups that merge
    # their residues in LDS: no partials, only the planned call's sequence order (64 int32) and its load-policy
    # flag (one int32), 256-B aligned.
    assert lib.sd_paged_decode_workspace_size(64, 5, 32, 8, 128, 256, 33) == 512
    assert lib.sd_paged_decode_workspace_size(63, 5, 32, 8, 128, 256, 33) == 256
    # 16 sequences: residue partials [16 items][8 heads][8 residues][32 rows] x (128 + 2) fp32
    assert lib.sd_paged_decode_workspace_size(16, 5, 32, 8, 128, 256, 33) >= 16 * 8 * 8 * 32 * 130 * 4
    # 9 queries x 4 heads = 36 rows -> 3 row tiles: merged in LDS at 64 sequences, partials at 16
    assert lib.sd_paged_decode_workspace_size(64, 9, 32, 8, 128, 256, 33) == 512
    assert lib.sd_paged_decode_workspace_size(16, 9, 32, 8, 128, 256, 33) >= 16 * 8 * 8 * 48 * 130 * 4
    # 17 queries x 4 heads = 68 rows -> 4 row tiles (64 rows) in two query groups, never merged in LDS
    assert lib.sd_paged_decode_workspace_size(64, 17, 32, 8, 128, 256, 33) >= 128 * 8 * 8 * 64 * 130 * 4
    assert lib.sd_paged_decode_workspace_size(0, 5, 32, 8, 128, 256, 33) == 0
    assert lib.sd_varlen_workspace_size(51, 2048, 4096, 32, 8, 128) > 0
    # per-row statistics of 6 spans (16 B each) for 64 x 5 target and 64 x 4 draft rows
    assert lib.sd_verify_workspace_size(64, 4, 151936, 1) >= (64 * 5 + 64 * 4) * 6 * 16
    # sd_linear, qkv shape (24 tiles, each split into 8 ranges): up to 320 rows the packed rows plus every
    # range's fp32 sums (one row of workgroups: 24 x 8 x 327,680 B); past it the ranges run in order in one
    # workgroup, so only the packed rows (1168 -> 1280 rows of 4096 bf16); not monotonic in the rows
    small, large = lib.sd_linear_workspace_size(320, 6144, 4096), lib.sd_linear_workspace_size(1168, 6144, 4096)
    assert small >= 320 * 4096 * 2 + 24 * 8 * 327680 and large == 1280 * 4096 * 2 and large < small
    # a vocabulary-sized projection keeps the physical split at any row count: sums for every row of workgroups
    assert lib.sd_linear_workspace_size(640, 151936, 4096) >= 640 * 4096 * 2 + 2 * 82 * 3 * 327680


def test_bad_arguments_return_status(lib):
    rc = lib.sd_store_kvcache(None, 0, None, 0, None, None, 0, None, -1, 8, 128, None)
    assert rc == 1 and b"bad sizes" in lib.sd_last_error()
    assert lib.sd_store_kvcache(None, 0, None, 0, None, None, 0, None, 0, 8, 128, None) == 0   # nothing to do
    rc = lib.sd_paged_decode(None, 4096, None, None, 10, 256, None, None, 4, 2, 5, 32, 8, 64, 0.1, None, 4096,
                             None, 0, None)
    assert rc == 2 and b"head_dim 64" in lib.sd_last_error()
    rc = lib.sd_paged_decode(None, 4096, None, None, 10, 100, None, None, 4, 2, 5, 32, 8, 128, 0.1, None, 4096,
                             None, 0, None)
    assert rc == 2 and b"block_size" in lib.sd_last_error()
    rc = lib.sd_paged_decode(None, 4096, None, None, 10, 32, None, None, 2049, 2, 5, 32, 8, 128, 0.1, None, 4096,
                             None, 0, None)
    assert rc == 2 and b"table width 2049 exceeds 2048" in lib.sd_last_error()
    rc = lib.sd_varlen_attention(None, 4096, None, 1024, None, 1024, 0, 0, 0, None, 0, None, None, 1, 10, 10, 10,
                                 30, 8, 128, 0.1, None, 4096, None, 0, None)
    assert rc == 1 and b"multiple" in lib.sd_last_error()
    rc = lib.sd_verify_drafts(None, 0, 10, None, None, None, None, 0, 0, None, None, 2, 70, 10, None, None, None, 0,
                              None)
    assert rc == 1
    ws = ctypes.create_string_buffer(16)
    rc = lib.sd_verify_drafts(ctypes.addressof(ws), 7, 10, ctypes.addressof(ws), ctypes.addressof(ws),
                              ctypes.addressof(ws), None, 0, 0, None, None, 2, 1, 10, ctypes.addressof(ws),
                              ctypes.addressof(ws), ctypes.addressof(ws), 16, None)
    assert rc == 2 and b"dtype" in lib.sd_last_error()
    nr = lib.sd_qk_norm_rope_store
    rc = nr(None, 4096, None, 1024, None, 1024, None, None, None, 1e-6, None, 100, None, 4096, None, 0, None, None,
            0, None, 4, 32, 8, 64, None)
    assert rc == 2 and b"head_dim 64" in lib.sd_last_error()
    rc = nr(None, 4096, None, 1024, None, 1024, None, ctypes.addressof(ws), None, 1e-6, None, 100, None, 4096, None,
            0, None, None, 0, None, 4, 32, 8, 128, None)
    assert rc == 1 and b"both norm weights" in lib.sd_last_error()
    rc = nr(None, 4096, None, 1024, None, 1024, None, None, None, 1e-6, None, 100, None, 4096, None, 0,
            ctypes.addressof(ws), None, 0, None, 4, 32, 8, 128, None)
    assert rc == 1 and b"store needs" in lib.sd_last_error()
    rc = nr(None, 4096, None, 1024, None, 1024, None, None, None, -1.0, None, 100, None, 4096, None, 0, None, None,
            0, None, 4, 32, 8, 128, None)
    assert rc == 1 and b"eps" in lib.sd_last_error()
    assert nr(None, 0, None, 0, None, 0, None, None, None, 1e-6, None, 100, None, 0, None, 0, None, None, 0, None,
              0, 32, 8, 128, None) == 0                                                    # nothing to do
    rc = lib.sd_linear(None, 4096, 4, None, 6144, 100, None, 6144, None, 0, None)
    assert rc == 2 and b"multiple of 32" in lib.sd_last_error()
    rc = lib.sd_linear(None, 4096, 4, None, 6144, 4096, None, 6144, None, 0, None)
    assert rc == 1 and b"null pointer" in lib.sd_last_error()
    assert lib.sd_linear(None, 0, 0, None, 6144, 4096, None, 0, None, 0, None) == 0            # nothing to do
    # packed rows [Mpad=64][4096] bf16, then [1 row of workgroups][16 split tiles][8 ranges] of fp32 sums
    assert lib.sd_linear_workspace_size(1, 4096, 4096) == 64 * 4096 * 2 + 16 * 8 * 8 * 2 * 1 * 16 * 64 * 4
    rn = lib.sd_rms_norm
    rc = rn(None, 4096, None, 0, None, 1e-6, 4, 4100, None, 4096, None, 0, None)
    assert rc == 2 and b"multiple of 8" in lib.sd_last_error()
    rc = rn(None, 4096, ctypes.addressof(ws), 4096, None, 1e-6, 4, 4096, None, 4096, None, 0, None)
    assert rc == 1 and b"together" in lib.sd_last_error()
    assert rn(None, 0, None, 0, None, 1e-6, 0, 4096, None, 0, None, 0, None) == 0                 # nothing to do
    di = lib.sd_draft_step_inputs
    rc = di(None, None, None, 33, 256, None, 5, 1, 4, None, None, None, None, None)
    assert rc == 1 and b"bad sizes" in lib.sd_last_error()                   # more tokens than sequences
    rc = di(None, None, None, 33, 256, None, 0, 1, 4, None, None, None, None, None)
    assert rc == 1 and b"null pointer" in lib.sd_last_error()
    assert di(None, None, None, 33, 256, None, 0, 1, 0, None, None, None, None, None) == 0  # nothing to do


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load()
