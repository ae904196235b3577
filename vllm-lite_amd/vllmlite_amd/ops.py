"""ctypes binding of the gfx950 C-ABI library (include/vllmlite_hip.h).

Device memory and streams come from PyTorch-ROCm; every call passes raw device
pointers and torch's current stream to the library. The library is loaded
after `import torch` so that it binds the HIP runtime torch already loaded
(both carry the soname libamdhip64.so.7). There is no fallback: if the
library is missing, `lib()` raises.
"""

from __future__ import annotations

import ctypes
import os
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from .build import LIB_PATH

# VL_DTYPE_*: F32_BF16KV / F32_FP8KV = fp32 query and out over bf16 / FP8 E4M3
# caches; FP8_E4M3 = OCP FP8 E4M3 cache elements (torch.float8_e4m3fn)
F32, BF16, F32_BF16KV, FP8_E4M3, F32_FP8KV = 0, 1, 2, 3, 4
# VL_KV_*: a per-layer cache tensor [slots, Hkv, D] is token-major (the
# reference's layout), [blocks, Hkv, block_size, D] head-major
KV_TOKEN_MAJOR, KV_HEAD_MAJOR = 0, 1
ABI_VERSION = 13  # vl_abi_version() of the library these signatures describe
_c_void_p = ctypes.c_void_p
_i32, _i64, _f32, _size = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes); must list every function of include/vllmlite_hip.h
SIGNATURES = {
    "vl_last_error": (ctypes.c_char_p, []),
    "vl_abi_version": (_i32, []),
    "vl_launcher_create": (_i32, [_i32, _c_void_p, ctypes.POINTER(_c_void_p)]),
    "vl_launcher_submit": (_i32, [_c_void_p, _c_void_p, _c_void_p, ctypes.POINTER(ctypes.c_uint64)]),
    "vl_launcher_wait": (_i32, [_c_void_p, ctypes.c_uint64]),
    "vl_launcher_destroy": (_i32, [_c_void_p]),
    "vl_host_wait_nonneg": (_i32, [_c_void_p, _i64, _i64]),
    "vl_reshape_and_cache": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p, _c_void_p,
                                    _c_void_p, _i64, _i32, _i32, _i32, _i32, _i32, _c_void_p]),
    "vl_copy_blocks": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i32, _i32, _i64, _i64, _i32,
                              _c_void_p]),
    "vl_paged_attention_workspace_size": (_size, [_i32, _i32, _i32, _i32, _i32]),
    "vl_paged_attention_min_workspace": (_size, [_i32]),
    "vl_paged_attention": (_i32, [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
                                  _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _i32, _i32, _i32,
                                  _f32, _i32, _i32, _i32, _i32, _i32, _c_void_p, _size,
                                  _c_void_p]),
    "vl_paged_attention_reads_plan": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "vl_paged_attention_plan": (_i32, [_c_void_p, _c_void_p, _i32, _i32, _i32, _i32, _i32, _i32,
                                       _i32, _c_void_p, _size, _c_void_p]),
    "vl_paged_attention_run": (_i32, [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p,
                                      _c_void_p, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32,
                                      _i32, _i32, _i32, _f32, _i32, _i32, _i32, _i32, _i32,
                                      _c_void_p, _size, _c_void_p]),
    "vl_paged_attention_noalloc": (_i32, [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p,
                                          _c_void_p, _i32, _c_void_p, _c_void_p, _i32, _i32,
                                          _i32, _i32, _i32, _i32, _f32, _i32, _i32, _i32,
                                          _i32, _i32, _c_void_p]),
    "vl_rms_norm": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _f32,
                           _c_void_p]),
    "vl_silu_mul": (_i32, [_c_void_p, _c_void_p, _i64, _i32, _c_void_p]),
    "vl_rope_and_cache": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                 _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i32, _i32, _i32,
                                 _i32, _i32, _c_void_p]),
    "vl_greedy_verify": (_i32, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p, _c_void_p, _i32,
                                _c_void_p, _c_void_p, _i32, _c_void_p, _i64, _c_void_p]),
    "vl_argmax_rows": (_i32, [_c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p, _c_void_p]),
    "vl_linear_rows": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _i64,
                              _c_void_p, _f32, _i32, _i32, _i32, _i32, _c_void_p]),
    "vl_qkv_rope_cache": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p,
                                 _c_void_p, _i64,
                                 _c_void_p, _c_void_p, _i64, _i32, _c_void_p, _f32, _c_void_p,
                                 _c_void_p, _c_void_p, _c_void_p, _i32, _i32, _i32, _i32, _i32,
                                 _i32, _i32, _i32, _c_void_p, _c_void_p, _i64, _c_void_p]),
    "vl_resolve_tokens": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p]),
    "vl_copy_words": (_i32, [_c_void_p, _c_void_p, _i64, _c_void_p]),
    "vl_linear_rows_argmax": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p,
                                     _c_void_p, _f32, _i32, _i32, _i32, _c_void_p, _c_void_p,
                                     _c_void_p, _i64, _c_void_p]),
    "vl_linear_rows_parts": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i32, _c_void_p,
                                    _c_void_p, _c_void_p, _f32, _i32, _i32, _i32, _c_void_p]),
    "vl_decode_attention_wo": (_i32, [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
                                      _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _i32, _i32,
                                      _f32, _i32, _i32, _i32, _c_void_p, _i32, _c_void_p]),
    "vl_decode_step_supported": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "vl_decode_step": (_i32, [_c_void_p, _c_void_p, _i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                              _c_void_p, _i64, _i32, _i32, _c_void_p, _c_void_p, _c_void_p,
                              _c_void_p, _c_void_p, _i32, _i32, _c_void_p, _i32, _c_void_p,
                              _c_void_p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _f32,
                              _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                              _c_void_p, _c_void_p, _c_void_p]),
}

_LIB: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"HIP library not built: {LIB_PATH} is missing "
                "(run `python -m vllmlite_amd.build` or __graft_entry__.build())")
        handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.vl_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {handle.vl_abi_version()}, these bindings "
                               f"need {ABI_VERSION}: rebuild the library")
        _LIB = handle
    return _LIB


_HIP = None


def hip_runtime():
    """The HIP runtime library torch has loaded, for the per-step launch path
    of HipRunner (hipGraphLaunch of a captured step, hipEventRecord /
    hipEventSynchronize, hipSetDevice) without torch's per-call overhead."""
    global _HIP
    if _HIP is None:
        h = ctypes.CDLL("libamdhip64.so")
        for name, args in (("hipGraphLaunch", [_c_void_p, _c_void_p]),
                           ("hipEventRecord", [_c_void_p, _c_void_p]),
                           ("hipEventSynchronize", [_c_void_p]),
                           ("hipSetDevice", [_i32]),
                           ("hipGetErrorString", [_i32])):
            fn = getattr(h, name)
            fn.argtypes = args
            fn.restype = _i32
        h.hipGetErrorString.restype = ctypes.c_char_p
        _HIP = h
    return _HIP


class Launcher:
    """vl_launcher_*: graph launches (and event records) submitted to a host
    thread of the library's, in order, on one stream."""

    def __init__(self, device: int, stream_handle: int):
        h = _c_void_p()
        _check(lib().vl_launcher_create(device, _c_void_p(stream_handle), ctypes.byref(h)),
               "vl_launcher_create")
        self._h = h
        self._t = ctypes.c_uint64()
        self.last = 0  # the last ticket handed out

    def submit(self, graph_exec: int, event: int = 0) -> int:
        _check(lib().vl_launcher_submit(self._h, _c_void_p(graph_exec), _c_void_p(event),
                                        ctypes.byref(self._t)), "vl_launcher_submit")
        self.last = self._t.value
        return self.last

    def wait(self, ticket: int) -> None:
        if ticket:
            _check(lib().vl_launcher_wait(self._h, ticket), "vl_launcher_wait")

    def drain(self) -> None:
        """Until every submission's calls have returned (before the caller
        itself enqueues work on the same stream)."""
        self.wait(self.last)

    def close(self) -> None:
        if self._h is not None and _LIB is not None:
            lib().vl_launcher_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def host_wait_nonneg(values: np.ndarray, timeout_s: float = 30.0) -> None:
    """Until every entry of a pinned int32 host array is >= 0 (written by a
    kernel after the caller set them negative); raises after timeout_s."""
    _need(values.dtype == np.int32 and values.flags.c_contiguous, "contiguous int32 array")
    _check(lib().vl_host_wait_nonneg(values.ctypes.data, values.size, int(timeout_s * 1e6)),
           "vl_host_wait_nonneg")


def hip_check(rc: int, what: str) -> None:
    if rc != 0:
        msg = hip_runtime().hipGetErrorString(rc).decode(errors="replace")
        raise RuntimeError(f"{what} failed (hipError {rc}): {msg}")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().vl_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.bfloat16:
        return BF16
    if t.dtype == torch.float8_e4m3fn:
        return FP8_E4M3
    raise TypeError(f"unsupported dtype {t.dtype}")


def _attn_dtype(query: torch.Tensor, cache: torch.Tensor) -> int:
    """VL_DTYPE_* of an attention call: the query's, or F32_BF16KV /
    F32_FP8KV for an fp32 query over bf16 / FP8 E4M3 caches."""
    if query.dtype == torch.float32 and cache.dtype == torch.bfloat16:
        return F32_BF16KV
    if query.dtype == torch.float32 and cache.dtype == torch.float8_e4m3fn:
        return F32_FP8KV
    return _dtype_code(query)


def _cache_dtype(key_cache: torch.Tensor, value_cache: torch.Tensor) -> int:
    _need(key_cache.dtype == value_cache.dtype and
          key_cache.dtype in (torch.float32, torch.bfloat16, torch.float8_e4m3fn),
          "caches must both be fp32, both bf16 or both float8_e4m3fn")
    return _dtype_code(key_cache)


def kv_layout(cache: torch.Tensor):
    """(VL_KV_* layout, num_kv_heads, block_size (0: token-major, any),
    head_dim) of one layer's cache tensor: [slots, Hkv, D] is token-major,
    [blocks, Hkv, block_size, D] head-major."""
    if cache.dim() == 3:
        return KV_TOKEN_MAJOR, cache.shape[1], 0, cache.shape[2]
    _need(cache.dim() == 4, "a layer's cache is [slots, Hkv, D] or [blocks, Hkv, block_size, D]")
    return KV_HEAD_MAJOR, cache.shape[1], cache.shape[2], cache.shape[3]


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _dev_i32(t: torch.Tensor, name: str) -> None:
    _need(t.is_cuda and t.dtype == torch.int32 and t.is_contiguous(),
          f"{name} must be a contiguous int32 device tensor")


# ------------------------------------------------------------------ K1 -----
def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                      value_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """key/value [T, Hkv, D] (rows may be strided), caches [slots, Hkv, D] or
    head-major [blocks, Hkv, block_size, D]."""
    T, hkv, d = key.shape
    _need(value.shape == key.shape, "key/value shapes differ")
    layout, c_hkv, bs, c_d = kv_layout(key_cache)
    _need((c_hkv, c_d) == (hkv, d) and value_cache.shape == key_cache.shape,
          "cache shape mismatch")
    _need(key_cache.is_contiguous() and value_cache.is_contiguous(), "caches must be contiguous")
    for t in (key, value):
        _need(t.stride(2) == 1 and t.stride(1) == d, "key/value rows must be [Hkv, D] contiguous")
    _need(key.dtype == value.dtype == key_cache.dtype == value_cache.dtype, "dtype mismatch")
    _dev_i32(slot_mapping, "slot_mapping")
    _need(slot_mapping.numel() == T, "slot_mapping length != tokens")
    _check(lib().vl_reshape_and_cache(_ptr(key), _ptr(value), key.stride(0), value.stride(0),
                                      _ptr(key_cache), _ptr(value_cache), _ptr(slot_mapping), T,
                                      hkv, d, _dtype_code(key), layout, bs, _stream()),
           "vl_reshape_and_cache")


# ------------------------------------------------------------------ K3 -----
def copy_blocks(key_cache: torch.Tensor, value_cache: torch.Tensor, block_pairs: torch.Tensor,
                block_size: int) -> None:
    """Caches [L, slots, Hkv, D] or head-major [L, blocks, Hkv, block_size, D]
    (a block is the same span in both); block_pairs int32 [n, 2] on the
    device."""
    _need(key_cache.is_contiguous() and value_cache.is_contiguous(), "caches must be contiguous")
    _need(key_cache.shape == value_cache.shape and key_cache.dim() in (4, 5),
          "cache shape mismatch")
    _need(key_cache.dim() == 4 or key_cache.shape[3] == block_size, "block_size mismatch")
    _dev_i32(block_pairs, "block_pairs")
    n = block_pairs.shape[0]
    L = key_cache.shape[0]
    layer = key_cache[0].numel()
    hkv, d = key_cache.shape[2], key_cache.shape[-1]
    _check(lib().vl_copy_blocks(_ptr(key_cache), _ptr(value_cache), _ptr(block_pairs), n, L,
                                layer, block_size * hkv * d, _dtype_code(key_cache),
                                _stream()),
           "vl_copy_blocks")


# ------------------------------------------------------------------ K2 -----
class AttentionWorkspace:
    """Reusable device scratch for paged_attention (grows on demand)."""

    def __init__(self, device=None):
        self.device = device
        self.buf: Optional[torch.Tensor] = None

    def get(self, nbytes: int) -> torch.Tensor:
        nbytes = max(256, (int(nbytes) + 255) // 256 * 256)
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.empty(nbytes, dtype=torch.uint8, device=self.device or "cuda")
        return self.buf


def paged_attention_workspace_size(num_seqs, num_tokens, num_heads, head_dim, max_context_len):
    return int(lib().vl_paged_attention_workspace_size(num_seqs, num_tokens, num_heads, head_dim,
                                                       max_context_len))


def _attn_check(out, query, key_cache, value_cache, block_tables, seq_lens, query_start_loc,
                workspace):
    T, H, D = query.shape
    _need(query.stride(2) == 1 and query.stride(1) == D, "query rows must be [H, D] contiguous")
    _need(out.shape == (T, H, D) and out.is_contiguous() and out.dtype == query.dtype,
          "out must be a contiguous [T, H, D] tensor of the query dtype")
    _need(key_cache.dim() in (3, 4) and key_cache.shape == value_cache.shape and
          key_cache.shape[-1] == D, "cache shape mismatch")
    _need(key_cache.is_contiguous() and value_cache.is_contiguous(), "caches must be contiguous")
    _need(key_cache.dtype == value_cache.dtype and
          (key_cache.dtype == query.dtype or
           (query.dtype == torch.float32 and
            key_cache.dtype in (torch.bfloat16, torch.float8_e4m3fn))),
          "dtype mismatch (caches of the query dtype, or bf16 / float8_e4m3fn under an "
          "fp32 query)")
    hkv = key_cache.shape[1]
    _need(H % hkv == 0, "num_heads must be a multiple of num_kv_heads")
    for t, n in ((block_tables, "block_tables"), (seq_lens, "seq_lens"),
                 (query_start_loc, "query_start_loc")):
        _dev_i32(t, n)
    S = seq_lens.numel()
    _need(query_start_loc.numel() == S + 1 and block_tables.dim() == 2 and
          block_tables.shape[0] == S, "metadata shapes disagree")
    _need(workspace.is_cuda and workspace.data_ptr() % 256 == 0, "workspace must be 256-aligned")
    return T, H, hkv, D, S


def _cache_layout(key_cache, block_size):
    layout, _, bs, _ = kv_layout(key_cache)
    _need(layout == KV_TOKEN_MAJOR or bs == block_size,
          "block_size differs from the head-major cache's block dimension")
    return layout


def _attn_args(out, query, key_cache, value_cache, block_tables, seq_lens, query_start_loc,
               scale, block_size, workspace, max_query_len, min_query_len, max_context_len,
               T, H, hkv, D, S):
    return (_ptr(out), _ptr(query), query.stride(0), _ptr(key_cache), _ptr(value_cache),
            _ptr(block_tables), block_tables.stride(0), _ptr(seq_lens), _ptr(query_start_loc),
            S, T, H, hkv, D, block_size, float(scale), _attn_dtype(query, key_cache),
            _cache_layout(key_cache, block_size), int(max_query_len), int(min_query_len),
            int(max_context_len), _ptr(workspace), workspace.numel() * workspace.element_size(),
            _stream())


def paged_attention(out: torch.Tensor, query: torch.Tensor, key_cache: torch.Tensor,
                    value_cache: torch.Tensor, block_tables: torch.Tensor, seq_lens: torch.Tensor,
                    query_start_loc: torch.Tensor, scale: float, block_size: int,
                    workspace: torch.Tensor, max_query_len: int = 0,
                    min_query_len: int = 0, max_context_len: int = 0) -> None:
    """query [T, H, D] (token rows may be strided), caches [slots, Hkv, D] or
    head-major [blocks, Hkv, block_size, D], block_tables int32 [S, W],
    seq_lens int32 [S], query_start_loc int32 [S+1].
    max_query_len / min_query_len: host-known bounds on the query count of
    the sequences that have queries, max_context_len on seq_lens (0 =
    unknown); they pick the launches."""
    dims = _attn_check(out, query, key_cache, value_cache, block_tables, seq_lens,
                       query_start_loc, workspace)
    _check(lib().vl_paged_attention(*_attn_args(out, query, key_cache, value_cache, block_tables,
                                                seq_lens, query_start_loc, scale, block_size,
                                                workspace, max_query_len, min_query_len,
                                                max_context_len, *dims)),
           "vl_paged_attention")


def paged_attention_plan(query: torch.Tensor, key_cache: torch.Tensor, seq_lens: torch.Tensor,
                         query_start_loc: torch.Tensor, block_size: int,
                         workspace: torch.Tensor) -> None:
    """Plan once per batch; reuse with paged_attention_run for every layer."""
    T, H, D = query.shape
    hkv = kv_layout(key_cache)[1]
    _dev_i32(seq_lens, "seq_lens")
    _dev_i32(query_start_loc, "query_start_loc")
    S = seq_lens.numel()
    _need(query_start_loc.numel() == S + 1, "query_start_loc length")
    _need(workspace.is_cuda and workspace.data_ptr() % 256 == 0, "workspace must be 256-aligned")
    _check(lib().vl_paged_attention_plan(_ptr(seq_lens), _ptr(query_start_loc), S, T, H, hkv, D,
                                         block_size, _attn_dtype(query, key_cache), _ptr(workspace),
                                         workspace.numel() * workspace.element_size(), _stream()),
           "vl_paged_attention_plan")


def paged_attention_reads_plan(num_heads: int, num_kv_heads: int, head_dim: int,
                               block_size: int, max_query_len: int = 0,
                               max_context_len: int = 0) -> bool:
    """Whether paged_attention_run with these shapes and hints reads the plan
    (False: the short-decode kernel, whose plan call may be skipped)."""
    return bool(lib().vl_paged_attention_reads_plan(num_heads, num_kv_heads, head_dim, block_size,
                                                    max_query_len, max_context_len))


def paged_attention_run(out, query, key_cache, value_cache, block_tables, seq_lens,
                        query_start_loc, scale, block_size, workspace,
                        max_query_len: int = 0, min_query_len: int = 0,
                        max_context_len: int = 0) -> None:
    dims = _attn_check(out, query, key_cache, value_cache, block_tables, seq_lens,
                       query_start_loc, workspace)
    _check(lib().vl_paged_attention_run(*_attn_args(out, query, key_cache, value_cache,
                                                    block_tables, seq_lens, query_start_loc,
                                                    scale, block_size, workspace, max_query_len,
                                                    min_query_len, max_context_len, *dims)),
           "vl_paged_attention_run")


NOALLOC_SCRATCH_BYTES = 32 << 20  # VL_NOALLOC_SCRATCH_BYTES


def paged_attention_noalloc(out, query, key_cache, value_cache, block_tables, seq_lens,
                            query_start_loc, scale, block_size, max_query_len: int = 0,
                            min_query_len: int = 0, max_context_len: int = 0) -> None:
    """paged_attention with the library's static per-GPU scratch as the
    workspace (vl_paged_attention_noalloc): nothing is allocated."""
    T, H, D = query.shape
    _need(query.stride(2) == 1 and query.stride(1) == D, "query rows must be [H, D] contiguous")
    _need(out.shape == (T, H, D) and out.is_contiguous() and out.dtype == query.dtype,
          "out must be a contiguous [T, H, D] tensor of the query dtype")
    _need(key_cache.dim() in (3, 4) and key_cache.shape == value_cache.shape,
          "cache shape mismatch")
    for t, n in ((block_tables, "block_tables"), (seq_lens, "seq_lens"),
                 (query_start_loc, "query_start_loc")):
        _dev_i32(t, n)
    S = seq_lens.numel()
    _check(lib().vl_paged_attention_noalloc(
        _ptr(out), _ptr(query), query.stride(0), _ptr(key_cache), _ptr(value_cache),
        _ptr(block_tables), block_tables.stride(0), _ptr(seq_lens), _ptr(query_start_loc), S, T,
        H, key_cache.shape[1], D, block_size, float(scale), _attn_dtype(query, key_cache),
        _cache_layout(key_cache, block_size), int(max_query_len), int(min_query_len),
        int(max_context_len), _stream()),
        "vl_paged_attention_noalloc")


# ------------------------------------------------------------------ K4 -----
def rms_norm(out: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5,
             residual: Optional[torch.Tensor] = None) -> None:
    """fp32 rows; with `residual`, residual += x first and the sum is normalised."""
    rows, dim = x.shape
    for t in (out, x, weight) + ((residual,) if residual is not None else ()):
        _need(t.is_contiguous() and t.dtype == torch.float32, "fp32 contiguous tensors required")
    _need(out.shape == x.shape and weight.numel() == dim, "shape mismatch")
    _need(residual is None or residual.shape == x.shape, "residual shape mismatch")
    _check(lib().vl_rms_norm(_ptr(out), _ptr(residual), _ptr(x), _ptr(weight), rows, dim,
                             float(eps), _stream()), "vl_rms_norm")


LINEAR_STORE, LINEAR_ACCUMULATE, LINEAR_SWIGLU = 0, 1, 2
LINEAR_TILES16 = 16  # mode flag: the weight is in 16-column tiles
WEIGHT_ROWS, WEIGHT_TILES16 = 0, 1
LINEAR_ROWS_MAX = 16 * 65535  # rows per vl_linear_rows / vl_qkv_rope_cache call (16-row tiles)


def tile16(w: torch.Tensor, halves: int = 1) -> torch.Tensor:
    """A [k, halves * n] weight (k a multiple of 16) as 16-column tiles
    [halves * ceil(n/16), k, 16] (zero past column n; with halves 2, the tiles
    of w[:, :n] then those of w[:, n:], the SwiGLU gate and up halves). Inside
    a tile, element (k, m) with k = 16 g + 4 j + s sits at flat position
    256 g + 4 (16 j + m) + s."""
    k, cols = w.shape
    _need(k % 16 == 0, "k must be a multiple of 16")
    n = cols // halves
    nt = -(-n // 16)
    parts = []
    for h in range(halves):
        p = torch.zeros(k, nt * 16, dtype=w.dtype, device=w.device)
        p[:, :n] = w[:, h * n:(h + 1) * n]
        t = p.view(k, nt, 16).permute(1, 0, 2)  # [nt, k, 16]: (k, m)
        t = t.reshape(nt, k // 16, 4, 4, 16).permute(0, 1, 2, 4, 3)  # (g, j, s, m) -> (g, j, m, s)
        parts.append(t.reshape(nt, k, 16))
    return torch.cat(parts).contiguous()


def _weight_layout(weight: torch.Tensor, k: int, n: int, halves: int):
    """(tiles?, row stride) of a row-major [k, >= halves*n] or tiled weight."""
    if weight.dim() == 3:
        _need(weight.is_contiguous() and weight.shape == (halves * -(-n // 16), k, 16),
              "tiled weight must be [halves * ceil(n/16), k, 16]")
        return True, 0
    _need(weight.shape[0] == k and weight.shape[1] >= halves * n and weight.stride(-1) == 1,
          "weight shape mismatch")
    return False, weight.stride(0)


def linear_rows(out: torch.Tensor, x: torch.Tensor, weight: torch.Tensor,
                norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-5,
                mode: int = LINEAR_STORE, row_index: Optional[torch.Tensor] = None) -> None:
    """out (=, += or SwiGLU of) f(x) @ weight for fp32 rows (16-row tiles); f is
    the RMSNorm times norm_weight when given; with row_index the input rows
    are x[row_index] (see vl_linear_rows)."""
    k = x.shape[1]
    rows = out.shape[0] if row_index is not None else x.shape[0]
    n = out.shape[1]
    _need(row_index is None or (row_index.dtype == torch.int32 and row_index.numel() >= rows),
          "row_index must hold int32 row numbers")
    for t in (out, x, weight) + ((norm_weight,) if norm_weight is not None else ()):
        _need(t.dtype == torch.float32 and t.stride(-1) == 1, "fp32 row-major tensors required")
    _need(out.shape[0] == rows, "shape mismatch")
    tiles, wstride = _weight_layout(weight, k, n, 2 if mode == LINEAR_SWIGLU else 1)
    _need(norm_weight is None or norm_weight.numel() == k, "norm weight shape mismatch")
    _check(lib().vl_linear_rows(_ptr(out), out.stride(0), _ptr(x), x.stride(0), _ptr(row_index),
                                _ptr(weight), wstride, _ptr(norm_weight), float(eps), rows, k, n,
                                mode | (LINEAR_TILES16 if tiles else 0), _stream()),
           "vl_linear_rows")


def qkv_rope_cache(q_out: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                   x: torch.Tensor, weight: torch.Tensor, norm_weight: Optional[torch.Tensor],
                   positions: torch.Tensor, slot_mapping: torch.Tensor, cos: torch.Tensor,
                   sin: torch.Tensor, num_heads: int, num_kv_heads: int, head_dim: int,
                   eps: float = 1e-5, row_index: Optional[torch.Tensor] = None,
                   x_out: Optional[torch.Tensor] = None,
                   prev_ids: Optional[torch.Tensor] = None,
                   record: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> None:
    """QKV projection of a step's rows fused with RoPE and the K/V scatter; with
    row_index the rows are x[row_index] (an index -(1 + i) < 0 stands for
    prev_ids[i], the previous step's id of its row i), copied to x_out when
    given; record = (src, dst): int32 words the same launch copies from src
    (pinned host memory, which row_index / positions / slot_mapping may view)
    to dst (see vl_qkv_rope_cache)."""
    k = x.shape[1]
    rows = q_out.shape[0]
    _need(row_index is not None or x.shape[0] >= rows, "x has too few rows")
    _need(x_out is None or (x_out.is_contiguous() and x_out.shape[1] == k), "x_out shape mismatch")
    for t in (q_out, x, weight, cos, sin):
        _need(t.dtype == torch.float32 and t.stride(-1) == 1, "fp32 row-major tensors required")
    _need(key_cache.is_contiguous() and value_cache.is_contiguous(), "caches must be contiguous")
    cdt = _cache_dtype(key_cache, value_cache)
    layout, c_hkv, bs, c_d = kv_layout(key_cache)
    _need((c_hkv, c_d) == (num_kv_heads, head_dim) and value_cache.shape == key_cache.shape,
          "cache shape")
    _need(positions.numel() >= rows and slot_mapping.numel() >= rows, "shape mismatch")
    tiles, wstride = _weight_layout(weight, k, (num_heads + 2 * num_kv_heads) * head_dim, 1)
    _need(prev_ids is None or (row_index is not None and prev_ids.dtype == torch.int32),
          "prev_ids needs row_index and must hold int32 ids")
    rsrc, rdst, nrec = None, None, 0
    if record is not None:
        rsrc, rdst = record
        _need(rsrc.dtype == rdst.dtype == torch.int32 and rsrc.is_contiguous() and
              rdst.is_contiguous() and rsrc.numel() == rdst.numel() and
              (rsrc.is_pinned() or rsrc.is_cuda) and rdst.is_cuda,
              "record: contiguous int32 source (pinned or device) and device destination")
        nrec = rsrc.numel()
    _check(lib().vl_qkv_rope_cache(_ptr(q_out), _ptr(key_cache), _ptr(value_cache), _ptr(x),
                                   x.stride(0), _ptr(row_index), _ptr(prev_ids),
                                   prev_ids.numel() if prev_ids is not None else 0,
                                   _ptr(x_out), _ptr(weight),
                                   wstride, WEIGHT_TILES16 if tiles else WEIGHT_ROWS,
                                   _ptr(norm_weight),
                                   float(eps), _ptr(positions), _ptr(slot_mapping), _ptr(cos),
                                   _ptr(sin), rows, k, num_heads, num_kv_heads, head_dim, cdt,
                                   layout, bs, _ptr(rsrc), _ptr(rdst), nrec, _stream()),
           "vl_qkv_rope_cache")


def silu_mul(out: torch.Tensor, gate_up: torch.Tensor) -> None:
    rows, two_f = gate_up.shape
    _need(out.shape == (rows, two_f // 2) and out.is_contiguous() and gate_up.is_contiguous(),
          "shape mismatch")
    _check(lib().vl_silu_mul(_ptr(out), _ptr(gate_up), rows, two_f // 2, _stream()),
           "vl_silu_mul")


def rope_and_cache(qkv: torch.Tensor, q_out: torch.Tensor, key_cache: torch.Tensor,
                   value_cache: torch.Tensor, positions: torch.Tensor, slot_mapping: torch.Tensor,
                   cos: torch.Tensor, sin: torch.Tensor, num_heads: int, num_kv_heads: int,
                   head_dim: int) -> None:
    T = qkv.shape[0]
    _need(qkv.stride(1) == 1 and qkv.shape[1] >= (num_heads + 2 * num_kv_heads) * head_dim,
          "qkv rows must hold q|k|v")
    _need(q_out.shape == (T, num_heads, head_dim) and q_out.is_contiguous(), "q_out shape")
    layout, c_hkv, bs, c_d = kv_layout(key_cache)
    _need((c_hkv, c_d) == (num_kv_heads, head_dim) and key_cache.is_contiguous() and
          value_cache.shape == key_cache.shape and value_cache.is_contiguous(), "cache shape")
    _need(qkv.dtype == q_out.dtype == torch.float32, "qkv and q_out are fp32")
    cdt = _cache_dtype(key_cache, value_cache)
    _dev_i32(positions, "positions")
    _dev_i32(slot_mapping, "slot_mapping")
    _need(cos.shape == sin.shape and cos.shape[1] == head_dim // 2, "rope table shape")
    _check(lib().vl_rope_and_cache(_ptr(qkv), qkv.stride(0), _ptr(q_out), _ptr(key_cache),
                                   _ptr(value_cache), _ptr(positions), _ptr(slot_mapping),
                                   _ptr(cos), _ptr(sin), T, num_heads, num_kv_heads, head_dim,
                                   cdt, layout, bs, _stream()), "vl_rope_and_cache")


# ------------------------------------------------------------------ K5 -----
_verify_scratch: Dict[int, torch.Tensor] = {}  # per stream: left zero by every call


def greedy_verify(logits: torch.Tensor, row_start: torch.Tensor, num_drafts: torch.Tensor,
                  drafts: torch.Tensor, out_tokens: torch.Tensor,
                  num_accepted: torch.Tensor, scratch: Optional[torch.Tensor] = None) -> None:
    """logits fp32 [R, V]; drafts int32 [S, K]; out_tokens int32 [S, K+1].
    scratch: int64 device tensor of at least S (K + 1) + ceil(S / 2) entries,
    zero before the first call (every call leaves it zero); by default one
    kept per stream (calls on one stream run in order, so they share it)."""
    _need(logits.dtype == torch.float32 and logits.stride(1) == 1, "logits must be fp32 rows")
    S, K = drafts.shape
    for t, n in ((row_start, "row_start"), (num_drafts, "num_drafts"), (drafts, "drafts"),
                 (out_tokens, "out_tokens"), (num_accepted, "num_accepted")):
        _dev_i32(t, n)
    _need(out_tokens.shape == (S, K + 1) and num_accepted.numel() == S and
          row_start.numel() == S and num_drafts.numel() == S, "shape mismatch")
    words = S * (K + 1) + (S + 1) // 2
    if scratch is None:
        key = torch.cuda.current_stream(logits.device).cuda_stream
        scratch = _verify_scratch.get(key)
        if scratch is None or scratch.numel() < words or scratch.device != logits.device:
            scratch = torch.zeros(max(words, 1024), dtype=torch.int64, device=logits.device)
            _verify_scratch[key] = scratch
    _need(scratch.dtype == torch.int64 and scratch.is_cuda and scratch.is_contiguous() and
          scratch.numel() >= words, "scratch must be a contiguous int64 device tensor")
    _check(lib().vl_greedy_verify(_ptr(logits), logits.stride(0), logits.shape[1],
                                  _ptr(row_start), _ptr(num_drafts), _ptr(drafts), K,
                                  _ptr(out_tokens), _ptr(num_accepted), S, _ptr(scratch),
                                  scratch.numel() * 8, _stream()),
           "vl_greedy_verify")


def argmax_rows(logits: torch.Tensor, out: torch.Tensor,
                host_out: Optional[torch.Tensor] = None) -> None:
    """out[r] = argmax of logits row r (ties to the lowest index); host_out, a
    pinned int32 CPU tensor of at least as many entries, receives the same ids
    from the same launch (no copy behind it); read it after the stream has
    passed the launch."""
    _need(logits.dtype == torch.float32 and logits.stride(1) == 1, "logits must be fp32 rows")
    _dev_i32(out, "out")
    _need(out.numel() == logits.shape[0], "out length")
    _need(host_out is None or (host_out.dtype == torch.int32 and host_out.is_pinned() and
                               host_out.is_contiguous() and host_out.numel() >= out.numel()),
          "host_out must be a pinned contiguous int32 tensor")
    _check(lib().vl_argmax_rows(_ptr(logits), logits.stride(0), logits.shape[0], logits.shape[1],
                                _ptr(out), _ptr(host_out), _stream()), "vl_argmax_rows")


def linear_rows_argmax(out: torch.Tensor, x: torch.Tensor, weight: torch.Tensor,
                       norm_weight: Optional[torch.Tensor], ids: torch.Tensor,
                       scratch: torch.Tensor, host_ids: Optional[torch.Tensor] = None,
                       row_index: Optional[torch.Tensor] = None, eps: float = 1e-5) -> None:
    """out = f(x[row_index]) @ weight (tiled; f the RMSNorm times norm_weight
    when given) and ids[r] = argmax of out row r (numpy's rule), also into
    host_ids (pinned) when given, from one launch. scratch: int64 [>= rows +
    1], zero before the first call and left zero by every call (see
    vl_linear_rows_argmax)."""
    k = x.shape[1]
    rows, n = out.shape
    _need(row_index is None or (row_index.dtype == torch.int32 and row_index.numel() >= rows),
          "row_index must hold int32 row numbers")
    for t in (out, x, weight) + ((norm_weight,) if norm_weight is not None else ()):
        _need(t.dtype == torch.float32 and t.stride(-1) == 1, "fp32 row-major tensors required")
    _need(row_index is not None or x.shape[0] >= rows, "x has too few rows")
    tiles, _ = _weight_layout(weight, k, n, 1)
    _need(tiles, "weight must be in 16-column tiles")
    _need(norm_weight is None or norm_weight.numel() == k, "norm weight shape mismatch")
    _dev_i32(ids, "ids")
    _need(ids.numel() >= rows, "ids length")
    _need(scratch.dtype == torch.int64 and scratch.is_cuda and scratch.is_contiguous(),
          "scratch must be a contiguous int64 device tensor")
    _need(host_ids is None or (host_ids.dtype == torch.int32 and host_ids.is_pinned() and
                               host_ids.is_contiguous() and host_ids.numel() >= rows),
          "host_ids must be a pinned contiguous int32 tensor")
    _check(lib().vl_linear_rows_argmax(_ptr(out), out.stride(0), _ptr(x), x.stride(0),
                                       _ptr(row_index), _ptr(weight), _ptr(norm_weight),
                                       float(eps), rows, k, n, _ptr(ids), _ptr(host_ids),
                                       _ptr(scratch), scratch.numel() * 8, _stream()),
           "vl_linear_rows_argmax")


def linear_rows_parts(out: torch.Tensor, x: torch.Tensor, x_parts: torch.Tensor,
                      weight: torch.Tensor, norm_weight: Optional[torch.Tensor] = None,
                      eps: float = 1e-5, x_out: Optional[torch.Tensor] = None) -> None:
    """out = SwiGLU(f(x + sum_p x_parts[:, p]) @ weight) with f the RMSNorm
    times norm_weight when given; weight in 16-column tiles (gate tiles then up
    tiles); x_parts [rows, P, k]; the summed rows also to x_out when given
    (vl_linear_rows_parts)."""
    rows, k = x.shape
    n = out.shape[1]
    _need(x_parts.dim() == 3 and x_parts.shape[0] >= rows and x_parts.shape[2] == k and
          x_parts.is_contiguous(), "x_parts must be [rows, P, k] contiguous")
    for t in (out, x, x_parts, weight) + tuple(t for t in (norm_weight, x_out) if t is not None):
        _need(t.dtype == torch.float32 and t.stride(-1) == 1, "fp32 row-major tensors required")
    _need(x_out is None or (x_out.is_contiguous() and x_out.shape[1] == k), "x_out shape")
    tiles, _ = _weight_layout(weight, k, n, 2)
    _need(tiles, "weight must be in 16-column tiles")
    _check(lib().vl_linear_rows_parts(_ptr(out), out.stride(0), _ptr(x), x.stride(0),
                                      _ptr(x_parts), x_parts.shape[1], _ptr(x_out), _ptr(weight),
                                      _ptr(norm_weight), float(eps), out.shape[0], k, n,
                                      _stream()), "vl_linear_rows_parts")


def decode_attention_wo(parts: torch.Tensor, query: torch.Tensor, key_cache: torch.Tensor,
                        value_cache: torch.Tensor, block_tables: torch.Tensor,
                        seq_lens: torch.Tensor, query_start_loc: torch.Tensor, scale: float,
                        block_size: int, wo: torch.Tensor, max_context_len: int) -> None:
    """parts[s, g, :] = (decode attention output of sequence s, KV head g's
    query heads) @ wo[those rows] (vl_decode_attention_wo); query [T, H, D]
    fp32 (sequence s's token at row query_start_loc[s]), S = seq_lens.numel()
    sequences, wo [H * D, d_model] row-major fp32, parts [S, Hkv, d_model]."""
    _, H, D = query.shape
    S = seq_lens.numel()
    _need(query_start_loc.numel() == S + 1, "query_start_loc must have S + 1 entries")
    layout, Hkv, bs, cd = kv_layout(key_cache)
    _need(cd == D and bs in (0, block_size), "cache shape")
    _need(query.dtype == torch.float32 and query.stride(-1) == 1 and query.stride(1) == D,
          "query must be fp32 [S, H, D] rows")
    _need(parts.dtype == torch.float32 and parts.is_contiguous() and
          parts.shape[0] >= S and parts.shape[1] == Hkv and parts.shape[2] == wo.shape[1],
          "parts must be [S, Hkv, d_model] fp32")
    _need(wo.dtype == torch.float32 and wo.is_contiguous() and wo.shape[0] == H * D, "wo shape")
    _need(block_tables.dtype == torch.int32 and block_tables.stride(-1) == 1, "int32 block tables")
    cdt = _cache_dtype(key_cache, value_cache)
    dtype = {BF16: F32_BF16KV, FP8_E4M3: F32_FP8KV}.get(cdt, F32)
    _check(lib().vl_decode_attention_wo(_ptr(parts), _ptr(query), query.stride(0),
                                        _ptr(key_cache), _ptr(value_cache), _ptr(block_tables),
                                        block_tables.stride(0), _ptr(seq_lens),
                                        _ptr(query_start_loc), S, H, Hkv, D, block_size,
                                        float(scale), dtype, layout, int(max_context_len),
                                        _ptr(wo), wo.shape[1], _stream()),
           "vl_decode_attention_wo")


def copy_words(dst: torch.Tensor, src: torch.Tensor) -> None:
    """dst[:] = src (int32, src may be pinned host memory) by one kernel
    (vl_copy_words)."""
    _need(dst.dtype == torch.int32 and src.dtype == torch.int32 and dst.is_contiguous() and
          src.is_contiguous() and dst.numel() == src.numel(), "int32 tensors of one size required")
    _check(lib().vl_copy_words(_ptr(dst), _ptr(src), dst.numel(), _stream()), "vl_copy_words")


def resolve_tokens(token_ids: torch.Tensor, prev_ids: torch.Tensor) -> None:
    """In place: ids t < 0 become prev_ids[-t - 1] (vl_resolve_tokens)."""
    _dev_i32(token_ids, "token_ids")
    _dev_i32(prev_ids, "prev_ids")
    _check(lib().vl_resolve_tokens(_ptr(token_ids), token_ids.numel(), _ptr(prev_ids),
                                   prev_ids.numel(), _stream()), "vl_resolve_tokens")


# ------------------------------------------------------------------ K7 -----
DECODE_STEP_ROWS = 16  # token rows (= sequences) of one vl_decode_step launch


def decode_step_supported(d_model: int, num_heads: int, num_kv_heads: int, d_ff: int,
                          kv_dtype: torch.dtype, max_context: int) -> bool:
    code = {torch.float32: F32, torch.bfloat16: BF16, torch.float8_e4m3fn: FP8_E4M3}.get(kv_dtype)
    if code is None:
        return False
    return bool(lib().vl_decode_step_supported(d_model, num_heads, num_kv_heads, d_ff, code,
                                               max_context))


class DecodeStep:
    """What vl_decode_step keeps between launches: the 6 weight buffers of
    the layers (attn_norm, tiled QKV, tiled wo, ffn_norm, tiled gate|up,
    tiled w_down, each [n_layers, ...] with a fixed layer stride, as
    model.tile_weights stacks them) as a host array of addresses and strides,
    and the launch's sync words (zero-filled here; every launch leaves them
    zero)."""

    FIELDS = ("attn_norm", "w_qkv_t", "wo_t", "ffn_norm", "w_gate_up_t", "w_down_t")

    def __init__(self, packed: dict, device):
        self.n_layers = len(packed["layers"])
        bufs = [packed["stacked"][f] for f in self.FIELDS]
        for b in bufs:
            _need(b.is_contiguous() and b.shape[0] == self.n_layers and b.dtype == torch.float32,
                  "stacked fp32 weights [n_layers, ...]")
        self._bufs = bufs
        self.addrs = (ctypes.c_void_p * 6)(*[b.data_ptr() for b in bufs])
        self.strides = (ctypes.c_int64 * 6)(*[b[0].numel() for b in bufs])
        self.sync = torch.zeros(128, dtype=torch.int32, device=device)
        _need(self.sync.data_ptr() % 128 == 0, "sync words must be 128-byte aligned")


def decode_step(ds: DecodeStep, tok_emb, final_norm, lm_head_t, key_cache, value_cache,
                token_ids, positions, slot_mapping, seq_lens, block_tables, prev_ids,
                cos, sin, num_heads: int, num_kv_heads: int, block_size: int, max_context: int,
                scale: float, eps: float, x, q, attn, act, logits, out_ids, out_ids_host) -> None:
    """One decode step of the model in one launch (vl_decode_step): rows are
    the first 16 of token_ids / positions / slot_mapping; sequences the rows of
    seq_lens / block_tables [num_seqs <= 16, W]; the argmax ids land in
    out_ids[:16] and the pinned out_ids_host[:16]; the caller zeroes
    out_ids_host[16], which is non-zero afterwards if the launch failed."""
    n_layers = ds.n_layers
    R = DECODE_STEP_ROWS
    _need(key_cache.shape == value_cache.shape and key_cache.shape[0] == n_layers and
          key_cache.is_contiguous() and value_cache.is_contiguous(),
          "caches must be contiguous [n_layers, ...]")
    cdt = _cache_dtype(key_cache, value_cache)
    layout, hkv, bs, hd = kv_layout(key_cache[0])
    _need(hkv == num_kv_heads and (bs in (0, block_size)), "cache shape")
    d = x.shape[1]
    d_ff = act.shape[1]
    vocab = logits.shape[1]
    for t, n in ((token_ids, "token_ids"), (positions, "positions"),
                 (slot_mapping, "slot_mapping"), (seq_lens, "seq_lens"),
                 (block_tables, "block_tables"), (prev_ids, "prev_ids"), (out_ids, "out_ids")):
        _dev_i32(t, n)
    _need(token_ids.numel() >= R and positions.numel() >= R and slot_mapping.numel() >= R and
          out_ids.numel() >= R, "16 rows of tokens, positions, slots and ids")
    _need(block_tables.dim() == 2 and block_tables.stride(1) == 1 and
          block_tables.shape[0] == seq_lens.numel() <= R, "block_tables [num_seqs, W]")
    for t in (x, q, attn, act, logits, tok_emb, final_norm, lm_head_t, cos, sin):
        _need(t.dtype == torch.float32 and t.is_contiguous(), "fp32 contiguous tensors")
    _need(x.shape[0] >= R and q.numel() >= R * d and attn.numel() >= R * d and
          act.shape[0] >= R and logits.shape[0] >= R and tok_emb.shape[1] == d,
          "row buffers of at least 16 rows")
    _need(out_ids_host.dtype == torch.int32 and out_ids_host.is_pinned() and
          out_ids_host.is_contiguous() and out_ids_host.numel() > R,
          "out_ids_host must be a pinned int32 tensor of at least 17 entries")
    _check(lib().vl_decode_step(
        ds.addrs, ds.strides, n_layers, _ptr(tok_emb), _ptr(final_norm), _ptr(lm_head_t),
        _ptr(key_cache), _ptr(value_cache), key_cache[0].numel(), cdt, layout, _ptr(token_ids),
        _ptr(positions), _ptr(slot_mapping), _ptr(seq_lens), _ptr(block_tables),
        block_tables.stride(0), seq_lens.numel(), _ptr(prev_ids), prev_ids.numel(), _ptr(cos),
        _ptr(sin), d, num_heads, num_kv_heads, d_ff, vocab, block_size, max_context,
        float(scale), float(eps), _ptr(x), _ptr(q), _ptr(attn), _ptr(act), _ptr(logits),
        _ptr(out_ids), _ptr(out_ids_host), _ptr(ds.sync), _stream()), "vl_decode_step")
