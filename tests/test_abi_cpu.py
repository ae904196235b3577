"""The C-ABI library loads without a GPU and exports exactly what
include/vllmlite_hip.h declares, and the ctypes table covers all of it."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vllmlite_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vl_\w+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared()
    for must in ("vl_reshape_and_cache", "vl_copy_blocks", "vl_paged_attention",
                 "vl_rms_norm", "vl_rope_and_cache", "vl_greedy_verify", "vl_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from vllmlite_amd.build import LIB_PATH
    if not os.path.exists(LIB_PATH):
        pytest.fail(f"{LIB_PATH} not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_signatures_cover_the_header():
    from vllmlite_amd.ops import SIGNATURES
    assert sorted(SIGNATURES) == declared()


def test_no_compute_without_gpu_needed_for_queries():
    """Size queries are host-only and callable without a device."""
    from vllmlite_amd.build import LIB_PATH
    lib = ctypes.CDLL(LIB_PATH)
    lib.vl_paged_attention_min_workspace.restype = ctypes.c_size_t
    lib.vl_paged_attention_workspace_size.restype = ctypes.c_size_t
    assert lib.vl_paged_attention_min_workspace(10) >= 256
    assert lib.vl_paged_attention_workspace_size(256, 256, 32, 128, 8192) > \
        lib.vl_paged_attention_min_workspace(256)
    lib.vl_abi_version.restype = ctypes.c_int
    assert lib.vl_abi_version() == 13


def test_reads_plan_names_the_short_decode_shapes():
    """The host-only rule for which runs read no plan: one query per sequence,
    a context bound <= 2048, head_dim 16/32/48/64, 1/2/4/8 query heads per KV
    head, a power-of-two block size; every other case reads the plan."""
    from vllmlite_amd.build import LIB_PATH
    lib = ctypes.CDLL(LIB_PATH)
    f = lib.vl_paged_attention_reads_plan
    f.restype = ctypes.c_int
    assert f(8, 4, 48, 16, 1, 512) == 0          # the TinyLlama decode step
    assert f(8, 1, 64, 1, 1, 2048) == 0
    assert f(4, 4, 16, 4, 1, 1) == 0
    assert f(8, 4, 48, 16, 0, 512) == 1          # query bound unknown
    assert f(8, 4, 48, 16, 2, 512) == 1          # multi-query sequences
    assert f(8, 4, 48, 16, 1, 0) == 1            # context bound unknown
    assert f(8, 4, 48, 16, 1, 2049) == 1         # too long for the staged table
    assert f(32, 8, 128, 16, 1, 512) == 1        # head_dim 128: the bandwidth kernel
    assert f(12, 4, 48, 16, 1, 512) == 1         # 3 query heads per KV head
    assert f(8, 4, 48, 12, 1, 512) == 1          # block size not a power of two
    assert f(8, 3, 48, 16, 1, 512) == 1          # heads not a multiple of KV heads
    assert f(8, 0, 48, 16, 1, 512) == 1


def test_hip_runner_refuses_to_run_without_a_gpu():
    """No CPU fallback: without a device the runner raises instead of computing."""
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from vllmlite_amd.config import EngineConfig
    from vllmlite_amd.hip_runner import HipRunner
    cfg = EngineConfig()
    with pytest.raises(RuntimeError):
        HipRunner(cfg.model, cfg.cache)


def test_engine_default_backend_is_the_hip_runner():
    from vllmlite_amd.config import EngineConfig
    from vllmlite_amd.runner import make_runner
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(RuntimeError):
        make_runner(EngineConfig())


def test_tile16_layout():
    """Tiled projection weights: element (k, m) of tile t, k = 16 g + 4 j + s,
    at flat position 256 g + 4 (16 j + m) + s; columns past n zero; with
    halves 2 the gate tiles precede the up tiles."""
    import torch
    from vllmlite_amd.ops import tile16
    k, n = 48, 20
    w = torch.arange(k * 2 * n, dtype=torch.float32).reshape(k, 2 * n)
    t = tile16(w, halves=2)
    assert t.shape == (4, k, 16)
    flat = t.reshape(4, -1)
    for h in range(2):
        for tt in range(2):
            for kk in range(k):
                g, j, s = kk // 16, (kk % 16) // 4, kk % 4
                for m in range(16):
                    col = tt * 16 + m
                    want = w[kk, h * n + col].item() if col < n else 0.0
                    assert flat[2 * h + tt, 256 * g + 4 * (16 * j + m) + s].item() == want
