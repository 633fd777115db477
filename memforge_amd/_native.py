"""ctypes binding of ``libmemforge_hip.so`` (the C ABI in ``include/memforge_hip.h``).

This module is the only place Python touches the device library. Every
function takes torch tensors that already live on the GPU, passes their data
pointers and element strides to the C entry point on torch's current stream,
and raises if the library is missing, a tensor is on the wrong device, or the
entry point returns an error status. There is no fallback path: the data path
runs on the MI355X or not at all.
"""

from __future__ import annotations

import ctypes
from collections import OrderedDict
from dataclasses import dataclass
from pathlib import Path
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

LIB_PATH = Path(__file__).resolve().with_name("libmemforge_hip.so")

MF_F32, MF_F16, MF_BF16 = 0, 1, 2
DTYPE_CODES = {torch.float32: MF_F32, torch.float16: MF_F16, torch.bfloat16: MF_BF16}

PLAN_ITEM_INTS = 12
PLAN_MERGE_INTS = 8
SLICE_INTS = 8
SLICE_MAX_TILES = 512
SLICE_MAX_SEGMENTS = 64
SLICE_MIN_TILES = 64
SLICE_WAVES_PER_CU = 4
# 16-key tiles one wave of a plan may cover (MF_MAX_ITEM_TILES in
# paged_attention.hip); a cooperative unit of four waves covers four times that
MAX_ITEM_TILES = 128
ENTRY_INTS = 6

PACK_TABLE_OVERFLOW = 1
PACK_NEGATIVE_POSITION = 2
PACK_DUPLICATE_SLOT = 4
PACK_BAD_ENTRY = 8
PACK_ROW_COUNT = 16
PACK_BLOCK_OUT_OF_POOL = 32

_c_int, _c_i64, _c_f32, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p

_SIGNATURES = {
    "mf_version": (ctypes.c_char_p, []),
    "mf_last_hip_error": (_c_int, []),
    "mf_status_string": (ctypes.c_char_p, [_c_int]),
    "mf_kv_write": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp, _c_int,
                             _c_i64, _c_i64, _c_i64, _c_int, _c_i64, _c_int, _c_int, _vp]),
    "mf_kv_gather": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_i64, _vp, _c_i64,
                              _vp, _vp, _c_int, _c_i64, _c_i64, _c_int, _c_int, _vp]),
    "mf_kv_copy_blocks": (_c_int, [_vp, _vp, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _vp,
                                   _c_int, _vp]),
    "mf_ragged_pack": (_c_int, [_vp, _c_int, _vp, _c_i64, _vp, _c_i64, _c_int, _c_int, _c_i64, _vp,
                                _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _vp]),
    "mf_paged_attention": (_c_int, [
        _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64,
        _c_int, _vp, _c_i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_int, _c_int,
        _c_int, _c_f32, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _c_i64, _vp, _vp]),
    "mf_paged_attention_counted": (_c_int, [
        _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64,
        _c_int, _vp, _c_i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_int, _c_int,
        _c_int, _c_f32, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _vp]),
    "mf_paged_attention_kv_write": (_c_int, [
        _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64,
        _c_int, _vp, _c_i64, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64,
        _c_int, _c_int, _c_int, _c_f32, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _vp]),
    "mf_paged_attention_noalloc": (_c_int, [
        _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64,
        _c_int, _vp, _c_i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_int, _c_int,
        _c_int, _c_f32, _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp]),
    "mf_attention_plan": (_c_int, [_c_int, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                   _vp, _c_i64, _vp, _c_i64, _vp]),
    "mf_attention_plan_slices": (_c_int, [_c_int, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                          _c_int, _vp, _c_i64, _vp, _c_i64, _vp]),
    "mf_paged_attention_slices": (_c_int, [
        _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64,
        _c_int, _vp, _c_i64, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_f32, _vp, _c_i64, _c_i64,
        _vp, _c_i64, _vp, _c_i64, _vp]),
    "mf_spec_verify_workspace_size": (_c_i64, [_c_int, _c_int]),
    "mf_spec_verify": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _c_i64, _c_i64, _vp, _c_int,
                                _c_i64, _c_i64, _c_f32, _c_int, _vp, _vp, _c_i64, _vp, _vp, _vp,
                                _vp, _vp, _c_i64, _vp]),
}

_LIB: Optional[ctypes.CDLL] = None


def exported_symbols() -> Tuple[str, ...]:
    return tuple(_SIGNATURES)


def lib() -> ctypes.CDLL:
    """The loaded device library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m memforge_amd._build` "
                "(memforge_amd has no CPU fallback)"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _LIB = handle
    return _LIB


class MemforgeHipError(RuntimeError):
    """A device entry point rejected its arguments or failed to launch."""


def _check(status: int, what: str) -> None:
    if status != 0:
        L = lib()
        msg = L.mf_status_string(status).decode()
        raise MemforgeHipError(f"{what}: {msg} (status {status}, hip error {L.mf_last_hip_error()})")


def _stream(device: Optional[torch.device] = None) -> int:
    """Raw handle of the current HIP stream of ``device`` (default: the current
    device) -- the stream torch's own kernels are queued on, also under
    ``torch.cuda.stream`` and graph capture. The raw query costs about 0.1 us
    against 3 us for building a ``torch.cuda.Stream`` object."""
    if device is None or device.index is None:
        return torch._C._cuda_getCurrentRawStream(torch.cuda.current_device())
    return torch._C._cuda_getCurrentRawStream(device.index)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def require_device(*tensors: Optional[torch.Tensor]) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError(
                f"memforge_amd runs on the GPU; got a tensor on {t.device} "
                "(there is no CPU path)"
            )


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


# --------------------------------------------------------------- pool views

@dataclass(frozen=True)
class PoolView:
    """One layer of a paged K or V pool as the C ABI addresses it."""

    k: torch.Tensor  # tensor whose data_ptr is the layer base
    v: torch.Tensor
    stride_block: int
    stride_slot: int
    stride_head: int
    block_size: int
    num_heads: int
    head_dim: int

    @property
    def num_blocks(self) -> int:
        return int(self.k.shape[0])

    @property
    def num_slots(self) -> int:
        """Token slots of the layer; the kernels skip slots outside [0, num_slots)."""
        return int(self.k.shape[0]) * self.block_size

    @staticmethod
    def from_bshd(k: torch.Tensor, v: torch.Tensor) -> "PoolView":
        """``(blocks, slots, heads, dim)`` -- one layer of PagedKVPool."""
        if k.shape != v.shape or k.stride() != v.stride() or k.dtype != v.dtype:
            raise ValueError("K and V pools must share shape, strides and dtype")
        if k.stride(-1) != 1:
            raise ValueError("pool head_dim axis must be contiguous")
        n, bs, h, d = k.shape
        return PoolView(k, v, k.stride(0), k.stride(1), k.stride(2), bs, h, d)

    @staticmethod
    def from_bhsd(k: torch.Tensor, v: torch.Tensor) -> "PoolView":
        """``(blocks, heads, slots, dim)`` -- PagedKVCache's per-head layout."""
        if k.shape != v.shape or k.stride() != v.stride() or k.dtype != v.dtype:
            raise ValueError("K and V pools must share shape, strides and dtype")
        if k.stride(-1) != 1:
            raise ValueError("pool head_dim axis must be contiguous")
        n, h, bs, d = k.shape
        return PoolView(k, v, k.stride(0), k.stride(2), k.stride(1), bs, h, d)


def same_layout(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Same shape and the same strides on every axis longer than one (the
    stride of a length-one axis is never used to address an element)."""
    return a.shape == b.shape and all(x == y for x, y, n in zip(a.stride(), b.stride(), a.shape) if n > 1)


def _rows_ok(t: torch.Tensor, name: str) -> None:
    if t.dim() != 3:
        raise ValueError(f"{name} must be a (tokens, heads, head_dim) view, got {tuple(t.shape)}")
    if t.stride(-1) != 1 and t.shape[-1] > 1:
        raise ValueError(f"{name} head_dim axis must be contiguous")


# ----------------------------------------------------------- KV write/gather

def kv_write(k_rows: torch.Tensor, v_rows: torch.Tensor, slots: torch.Tensor, pool: PoolView) -> None:
    """Scatter (T, H, D) rows into pool slots ``slots`` (int64, device)."""
    _rows_ok(k_rows, "k_rows")
    _rows_ok(v_rows, "v_rows")
    if not same_layout(k_rows, v_rows):
        v_rows = v_rows.contiguous()
        k_rows = k_rows.contiguous()
    require_device(k_rows, v_rows, slots, pool.k)
    if slots.dtype != torch.int64 or not slots.is_contiguous():
        slots = slots.to(torch.int64).contiguous()
    T, H, D = k_rows.shape
    if H != pool.num_heads or D != pool.head_dim or slots.numel() != T:
        raise ValueError(
            f"rows {tuple(k_rows.shape)} / {slots.numel()} slots do not match a pool of "
            f"{pool.num_heads} heads x {pool.head_dim}"
        )
    _check(lib().mf_kv_write(
        _ptr(k_rows), _ptr(v_rows), dtype_code(k_rows.dtype), k_rows.stride(0), k_rows.stride(1),
        _ptr(slots), T, _ptr(pool.k), _ptr(pool.v), dtype_code(pool.k.dtype),
        pool.stride_block, pool.stride_slot, pool.stride_head, pool.block_size, pool.num_slots, H, D,
        _stream(k_rows.device),
    ), "mf_kv_write")


def kv_gather(pool: PoolView, slots: torch.Tensor, k_rows: torch.Tensor, v_rows: torch.Tensor) -> None:
    """Copy pool slots ``slots`` into preallocated (T, H, D) rows."""
    _rows_ok(k_rows, "k_rows")
    _rows_ok(v_rows, "v_rows")
    if not same_layout(k_rows, v_rows):
        raise ValueError("k_rows and v_rows must share strides")
    require_device(k_rows, v_rows, slots, pool.k)
    if slots.dtype != torch.int64 or not slots.is_contiguous():
        slots = slots.to(torch.int64).contiguous()
    T, H, D = k_rows.shape
    _check(lib().mf_kv_gather(
        _ptr(pool.k), _ptr(pool.v), dtype_code(pool.k.dtype), pool.stride_block, pool.stride_slot,
        pool.stride_head, pool.block_size, pool.num_slots, _ptr(slots), T, _ptr(k_rows), _ptr(v_rows),
        dtype_code(k_rows.dtype), k_rows.stride(0), k_rows.stride(1), H, D, _stream(k_rows.device),
    ), "mf_kv_gather")


def kv_copy_blocks(key_pool: torch.Tensor, value_pool: torch.Tensor,
                   pairs: Sequence[Tuple[int, int]]) -> None:
    """Copy block ``src`` to ``dst`` for every pair, in every layer of the
    ``(layers, blocks, slots, heads, dim)`` K and V pools (one launch per 32
    pairs; the pairs go in the kernel arguments)."""
    if key_pool.dim() != 5 or key_pool.shape != value_pool.shape:
        raise ValueError("block copy needs (layers, blocks, slots, heads, dim) K and V pools")
    if key_pool.stride() != value_pool.stride() or key_pool.dtype != value_pool.dtype:
        raise ValueError("K and V pools must share strides and dtype")
    L, N, bs, H, D = key_pool.shape
    if key_pool.stride()[2:] != (H * D, D, 1):
        raise ValueError("each block of a pool layer must be contiguous")
    require_device(key_pool, value_pool)
    flat = np.ascontiguousarray(np.asarray(list(pairs), dtype=np.int64).reshape(-1, 2))
    _check(lib().mf_kv_copy_blocks(
        _ptr(key_pool), _ptr(value_pool), dtype_code(key_pool.dtype), L, key_pool.stride(0),
        key_pool.stride(1), bs * H * D, N, flat.ctypes.data, flat.shape[0], _stream(key_pool.device),
    ), "mf_kv_copy_blocks")


# ------------------------------------------------------------------ uploads

def _layout(parts: Sequence[np.ndarray]) -> Tuple[List[np.ndarray], List[int], int]:
    """Contiguous copies of the parts, each part's int32-word offset (even, so
    int64 parts land on 8-byte boundaries) and the total word count."""
    arrs, offs, n = [], [], 0
    for p in parts:
        a = np.ascontiguousarray(p)
        if a.dtype not in (np.int32, np.int64):
            raise TypeError(f"upload takes int32/int64 arrays, got {a.dtype}")
        n = (n + 1) & ~1
        offs.append(n)
        n += a.size * a.itemsize // 4
        arrs.append(a)
    return arrs, offs, max(n, 2)


def _views(buf: torch.Tensor, arrs: Sequence[np.ndarray], offs: Sequence[int]) -> List[torch.Tensor]:
    out = []
    for a, o in zip(arrs, offs):
        t = buf[o:o + a.size * a.itemsize // 4]
        if a.dtype == np.int64:
            t = t.view(torch.int64)
        out.append(t.view(a.shape))
    return out


def _pack_host(parts: Sequence[np.ndarray], pinned: bool) -> Tuple[torch.Tensor, List[np.ndarray], List[int]]:
    """The parts packed into one int32 host tensor (pinned if asked), each on
    an 8-byte boundary: (tensor, contiguous parts, word offsets)."""
    arrs, offs, n = _layout(parts)
    host = torch.empty(n, dtype=torch.int32, pin_memory=pinned)
    h = host.numpy()
    for a, o in zip(arrs, offs):
        h[o:o + a.size * a.itemsize // 4] = a.reshape(-1).view(np.int32)
    return host, arrs, offs


def _refuse_capture(device: torch.device) -> None:
    """Uploads stage through a temporary pinned buffer that a captured copy
    would read again on every replay, after torch's host allocator has handed
    it out again; torch's pinned allocation is not permitted under capture
    anyway. Captured steps stage through buffers of their own
    (GraphedPagedDecoder, CountedPlan)."""
    if device.type == "cuda" and torch.cuda.is_current_stream_capturing():
        raise MemforgeHipError("host arrays cannot be uploaded under graph capture: stage them through "
                               "persistent buffers (GraphedPagedDecoder, CountedPlan) and capture those")


def upload_packed(parts: Sequence[np.ndarray], device) -> Tuple[torch.Tensor, List[int]]:
    """``upload`` without the per-part views: the device int32 buffer and each
    part's word offset in it (for callers that pass addresses to the C ABI)."""
    _refuse_capture(torch.device(device))
    host, _, offs = _pack_host(parts, True)
    buf = torch.empty(host.numel(), dtype=torch.int32, device=device)
    buf.copy_(host, non_blocking=True)
    return buf, offs


# upload_packed_cached: device buffers by their exact contents, device and
# stream, most recent last
_UPLOAD_CACHE: "OrderedDict[tuple, Tuple[torch.Tensor, List[int]]]" = OrderedDict()
UPLOAD_CACHE_SIZE = 64
UPLOAD_CACHE_MAX_WORDS = 1 << 18  # 1 MiB: at most 64 MiB of device memory held


def upload_packed_cached(parts: Sequence[np.ndarray], device) -> Tuple[torch.Tensor, List[int]]:
    """``upload_packed`` that hands back the buffer an earlier call made from
    the same bytes on the same device and stream (a model calling the
    attention operator once per layer sends the same tables, plan and
    positions for every layer of a step). The kernels only read these
    buffers, so sharing one between launches on its stream is safe; the key
    holds the stream, so no buffer is read on a stream its upload was not
    ordered before. Refused under graph capture, like every upload."""
    dev = torch.device(device)
    arrs, offs, words = _layout(parts)
    _refuse_capture(dev)  # a cached buffer could be evicted while a graph still replays
    if words > UPLOAD_CACHE_MAX_WORDS:  # a large launch amortises its own upload
        return upload_packed(arrs, dev)
    key = (dev.type, dev.index, _stream(dev) if dev.type == "cuda" else 0,
           tuple((a.dtype.str, a.shape) for a in arrs), b"".join(a.tobytes() for a in arrs))
    hit = _UPLOAD_CACHE.get(key)
    if hit is not None:
        _UPLOAD_CACHE.move_to_end(key)
        return hit
    made = upload_packed(arrs, dev)
    _UPLOAD_CACHE[key] = made
    if len(_UPLOAD_CACHE) > UPLOAD_CACHE_SIZE:
        _UPLOAD_CACHE.popitem(last=False)
    return made


def upload(parts: Sequence[np.ndarray], device) -> List[torch.Tensor]:
    """Move int32 / int64 host arrays to ``device`` with ONE host-to-device
    copy: they are packed into a pinned buffer (each part on an 8-byte
    boundary), copied asynchronously into a fresh device buffer on the current
    stream, and handed back as views with their own dtype and shape. The
    pinned buffer comes from torch's caching host allocator, which does not
    hand it out again before the copy has completed, so the host never waits
    for the GPU here."""
    dev = torch.device(device)
    _refuse_capture(dev)
    pinned = dev.type == "cuda"
    host, arrs, offs = _pack_host(parts, pinned)
    if not pinned:
        return _views(host.to(dev), arrs, offs)
    buf = torch.empty(host.numel(), dtype=torch.int32, device=dev)
    buf.copy_(host, non_blocking=True)
    return _views(buf, arrs, offs)


# ---------------------------------------------------------------- attention

@dataclass
class AttentionPlan:
    """Work list for one mf_paged_attention call (valid for its dtype/head_dim)."""

    items: torch.Tensor      # int32 device, (n_items, PLAN_ITEM_INTS); slice plans: (n_slices + n_segments, SLICE_INTS)
    merges: torch.Tensor     # int32 device, (n_merges, PLAN_MERGE_INTS)
    n_narrow: int            # slice plans: slices
    n_wide: int              # slice plans: segments
    n_merges: int
    partials_floats: int
    items_host: np.ndarray
    merges_host: np.ndarray
    sliced: bool = False     # a decode slice plan (mf_attention_plan_slices)


def plan_attention_host(cu_seqlens: Sequence[int], kv_lens: Sequence[int], num_q_heads: int,
                        num_kv_heads: int, head_dim: int, dtype: torch.dtype,
                        partition_tiles: int = 0) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """mf_attention_plan on host arrays: (items [n, PLAN_ITEM_INTS], merges
    [m, PLAN_MERGE_INTS], counts [n_narrow, n_wide, n_merges, partials_floats])."""
    cu = np.ascontiguousarray(np.asarray(cu_seqlens, dtype=np.int32))
    kv = np.ascontiguousarray(np.asarray(kv_lens, dtype=np.int32))
    B = kv.shape[0]
    if cu.shape[0] != B + 1:
        raise ValueError("cu_seqlens must have one more entry than kv_lens")
    counts = np.zeros(4, dtype=np.int64)
    L = lib()
    args = (B, cu.ctypes.data, kv.ctypes.data, num_q_heads, num_kv_heads, head_dim,
            dtype_code(dtype), partition_tiles)
    # One planner call when the plan fits the largest one seen so far (the
    # planner fills every row it reports); otherwise it reports the sizes and
    # a second call fills arrays of exactly that size.
    cap_items, cap_merges = _PLAN_CAPACITY
    items = np.empty((cap_items, PLAN_ITEM_INTS), dtype=np.int32)
    merges = np.empty((cap_merges, PLAN_MERGE_INTS), dtype=np.int32)
    st = L.mf_attention_plan(*args, items.ctypes.data, cap_items, merges.ctypes.data, cap_merges,
                             counts.ctypes.data)
    if st == -3:  # MF_ERR_WORKSPACE: counts holds the sizes
        n_items, n_merges = int(counts[0] + counts[1]), int(counts[2])
        _PLAN_CAPACITY[0] = max(cap_items, min(n_items, 1 << 16))
        _PLAN_CAPACITY[1] = max(cap_merges, min(n_merges, 1 << 14))
        items = np.empty((max(n_items, 1), PLAN_ITEM_INTS), dtype=np.int32)
        merges = np.empty((max(n_merges, 1), PLAN_MERGE_INTS), dtype=np.int32)
        st = L.mf_attention_plan(*args, items.ctypes.data, n_items, merges.ctypes.data, n_merges,
                                 counts.ctypes.data)
    _check(st, "mf_attention_plan")
    n_items = int(counts[0] + counts[1])
    n_merges = int(counts[2])
    return items[:n_items], merges[:n_merges], counts


# host array sizes for a one-call plan, grown to the largest plan seen
_PLAN_CAPACITY = [256, 64]


def plan_upload_parts(items: np.ndarray, merges: np.ndarray) -> List[np.ndarray]:
    """The two arrays a plan puts on the device (at least one row each)."""
    return [items if items.shape[0] else np.zeros((1, PLAN_ITEM_INTS), np.int32),
            merges if merges.shape[0] else np.zeros((1, PLAN_MERGE_INTS), np.int32)]


def plan_from_parts(items: np.ndarray, merges: np.ndarray, counts: np.ndarray,
                    dev_items: torch.Tensor, dev_merges: torch.Tensor, sliced: bool = False) -> AttentionPlan:
    return AttentionPlan(dev_items, dev_merges, int(counts[0]), int(counts[1]), int(counts[2]),
                         int(counts[3]), items, merges, sliced)


def plan_slices_host(cu_seqlens: Sequence[int], kv_lens: Sequence[int], num_q_heads: int,
                     num_kv_heads: int, head_dim: int, dtype: torch.dtype, num_cus: int,
                     min_tiles: int = SLICE_MIN_TILES) -> Optional[Tuple[np.ndarray, np.ndarray, np.ndarray]]:
    """mf_attention_plan_slices on host arrays for a GPU of ``num_cus``
    compute units: (slices [n_slices + n_segments, SLICE_INTS], merges [m,
    PLAN_MERGE_INTS], counts [n_slices, n_segments, n_merges,
    partials_floats]), or None when the launch does not qualify (not a pure
    decode step, or fewer than ``min_tiles`` tiles per wave of one round)."""
    cu = np.ascontiguousarray(np.asarray(cu_seqlens, dtype=np.int32))
    kv = np.ascontiguousarray(np.asarray(kv_lens, dtype=np.int32))
    B = kv.shape[0]
    if cu.shape[0] != B + 1:
        raise ValueError("cu_seqlens must have one more entry than kv_lens")
    counts = np.zeros(4, dtype=np.int64)
    L = lib()
    args = (B, cu.ctypes.data, kv.ctypes.data, num_q_heads, num_kv_heads, head_dim, dtype_code(dtype),
            int(num_cus), int(min_tiles))
    st = L.mf_attention_plan_slices(*args, None, 0, None, 0, counts.ctypes.data)
    if st == -2:  # MF_ERR_UNSUPPORTED: not a decode step this plan form serves
        return None
    if st not in (0, -3):
        _check(st, "mf_attention_plan_slices")
    if counts[0] == 0:
        return None
    n_rec, n_merges = int(counts[0] + counts[1]), int(counts[2])
    slices = np.empty((n_rec, SLICE_INTS), dtype=np.int32)
    merges = np.empty((max(n_merges, 1), PLAN_MERGE_INTS), dtype=np.int32)
    _check(L.mf_attention_plan_slices(*args, slices.ctypes.data, n_rec, merges.ctypes.data, n_merges,
                                      counts.ctypes.data), "mf_attention_plan_slices")
    return slices, merges[:n_merges], counts


_DEVICE_CUS = {}


def device_cus(device) -> int:
    """Compute units of ``device`` (a slice plan's size is set by it)."""
    dev = torch.device(device)
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    cus = _DEVICE_CUS.get(index)
    if cus is None:
        cus = _DEVICE_CUS[index] = torch.cuda.get_device_properties(index).multi_processor_count
    return cus


# plan_host results by their inputs, most recent last. The planners are pure
# functions of them, and a model that calls the attention operator once per
# layer asks for the same plan in every layer of a step. The arrays are handed
# out read-only, so no caller can change what a later hit returns.
_PLAN_CACHE: "OrderedDict[tuple, tuple]" = OrderedDict()
PLAN_CACHE_SIZE = 64


def plan_host(cu_seqlens: Sequence[int], kv_lens: Sequence[int], num_q_heads: int, num_kv_heads: int,
              head_dim: int, dtype: torch.dtype, device=None, partition_tiles: int = 0,
              decode_slices: bool = False) -> Tuple[np.ndarray, np.ndarray, np.ndarray, bool]:
    """Host plan arrays (items or slices, merges, counts) and whether they are
    a slice plan. With ``decode_slices`` (the caller's launch has 16-token
    blocks, no row map and no in-flight keys) a decode step large enough to
    fill the GPU on ``device`` more than once gets a slice plan; every other
    call, and an explicit ``partition_tiles``, the per-range plan."""
    slices = decode_slices and partition_tiles <= 0 and device is not None and torch.device(device).type == "cuda"
    cus = device_cus(device) if slices else 0
    key = (tuple(int(x) for x in cu_seqlens), tuple(int(x) for x in kv_lens), num_q_heads, num_kv_heads,
           head_dim, dtype, partition_tiles, cus)
    hit = _PLAN_CACHE.get(key)
    if hit is not None:
        _PLAN_CACHE.move_to_end(key)
        return hit
    made = plan_slices_host(cu_seqlens, kv_lens, num_q_heads, num_kv_heads, head_dim, dtype, cus) if slices else None
    if made is not None:
        out = (*made, True)
    else:
        out = (*plan_attention_host(cu_seqlens, kv_lens, num_q_heads, num_kv_heads, head_dim, dtype,
                                    partition_tiles), False)
    for a in out[:3]:
        a.flags.writeable = False
    _PLAN_CACHE[key] = out
    if len(_PLAN_CACHE) > PLAN_CACHE_SIZE:
        _PLAN_CACHE.popitem(last=False)
    return out


def plan_attention(cu_seqlens: Sequence[int], kv_lens: Sequence[int], num_q_heads: int,
                   num_kv_heads: int, head_dim: int, dtype: torch.dtype, device,
                   partition_tiles: int = 0, decode_slices: bool = False) -> AttentionPlan:
    """A plan for ``paged_attention`` (``plan_host``, then one upload)."""
    items, merges, counts, sliced = plan_host(cu_seqlens, kv_lens, num_q_heads, num_kv_heads, head_dim, dtype,
                                              device, partition_tiles, decode_slices)
    dev_items, dev_merges = upload(plan_upload_parts(items, merges), device)
    return plan_from_parts(items, merges, counts, dev_items, dev_merges, sliced)


class CountedPlan:
    """Fixed device buffers for a plan whose counts live in device memory
    (mf_paged_attention_counted): the shapes and addresses a captured HIP
    graph recorded stay valid while ``update`` swaps in each step's plan.

    Items hold ``cap_narrow`` narrow then ``cap_wide`` wide rows, each
    capacity rounded up to whole workgroups of four (the launch's grid, whose
    waves read their items before the live-count check); ``update`` raises if
    a plan does not fit. Host staging is pinned; each update waits for the
    previous one's copies before reusing it."""

    def __init__(self, cap_narrow: int, cap_wide: int, cap_merges: int, partials_floats: int, device):
        cap_narrow, cap_wide = -(-cap_narrow // 4) * 4, -(-cap_wide // 4) * 4
        self.cap_narrow, self.cap_wide, self.cap_merges = cap_narrow, cap_wide, cap_merges
        rows = max(cap_narrow + cap_wide, 1)
        self.items = torch.zeros((rows, PLAN_ITEM_INTS), dtype=torch.int32, device=device)
        self.merges = torch.zeros((max(cap_merges, 1), PLAN_MERGE_INTS), dtype=torch.int32, device=device)
        self.counts = torch.zeros(3, dtype=torch.int32, device=device)
        self.partials = torch.empty(max(partials_floats, 1), dtype=torch.float32, device=device)
        self._h_items = torch.zeros((rows, PLAN_ITEM_INTS), dtype=torch.int32).pin_memory()
        self._h_merges = torch.zeros((max(cap_merges, 1), PLAN_MERGE_INTS), dtype=torch.int32).pin_memory()
        self._h_counts = torch.zeros(3, dtype=torch.int32).pin_memory()
        self._copied = None

    def update(self, items: np.ndarray, merges: np.ndarray, counts: np.ndarray) -> None:
        n_narrow, n_wide, n_merges, floats = (int(x) for x in counts)
        if n_narrow > self.cap_narrow or n_wide > self.cap_wide or n_merges > self.cap_merges:
            raise ValueError(f"plan ({n_narrow}, {n_wide}, {n_merges}) exceeds the capacity "
                             f"({self.cap_narrow}, {self.cap_wide}, {self.cap_merges})")
        if floats > self.partials.numel():
            raise ValueError(f"plan needs {floats} partial floats, the buffer holds {self.partials.numel()}")
        if self._copied is not None:
            self._copied.synchronize()
        hi = self._h_items.numpy()
        hi[:n_narrow] = items[:n_narrow]
        hi[self.cap_narrow:self.cap_narrow + n_wide] = items[n_narrow:n_narrow + n_wide]
        if n_merges:
            self._h_merges.numpy()[:n_merges] = merges[:n_merges]
        self._h_counts.numpy()[:] = (n_narrow, n_wide, n_merges)
        self.items.copy_(self._h_items, non_blocking=True)
        if n_merges:
            self.merges[:n_merges].copy_(self._h_merges[:n_merges], non_blocking=True)
        self.counts.copy_(self._h_counts, non_blocking=True)
        self._copied = torch.cuda.Event()
        self._copied.record()


class Workspace:
    """Grow-only scratch for split-K partials (fp32), merge arrival counters
    (int32, kept all-zero between calls by the kernels) and the rejection
    verify, one per (device, stream) so concurrent streams never share it."""

    def __init__(self) -> None:
        self._partials = {}
        self._counters = {}
        self._verify = {}

    def partials(self, floats: int, device) -> Optional[torch.Tensor]:
        if floats <= 0:
            return None
        dev = torch.device(device)
        key = (dev.index, _stream(dev))
        buf = self._partials.get(key)
        if buf is None or buf.numel() < floats:
            buf = torch.empty(max(floats, 1 << 16), dtype=torch.float32, device=device)
            self._partials[key] = buf
        return buf

    def verify(self, nbytes: int, device, stream: Optional[int] = None) -> torch.Tensor:
        """mf_spec_verify's scratch, kept between calls (``stream``: the raw
        handle of the device's current stream, when the caller has it)."""
        dev = device if isinstance(device, torch.device) else torch.device(device)
        key = (dev.index, _stream(dev) if stream is None else stream)
        buf = self._verify.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            self._verify[key] = buf
        return buf

    def counters(self, n: int, device) -> Optional[torch.Tensor]:
        if n <= 0:
            return None
        dev = torch.device(device)
        key = (dev.index, _stream(dev))
        buf = self._counters.get(key)
        if buf is None or buf.numel() < n:
            buf = torch.zeros(max(n, 1 << 12), dtype=torch.int32, device=device)
            self._counters[key] = buf
        return buf


_WORKSPACE = Workspace()


def paged_attention(q_rows: torch.Tensor, out_rows: torch.Tensor, pool: PoolView,
                    block_tables: torch.Tensor, cu_seqlens: torch.Tensor, kv_lens: torch.Tensor,
                    positions: torch.Tensor, plan: AttentionPlan, scale: float,
                    num_kv_heads: int, row_map: Optional[torch.Tensor] = None,
                    pool_lens: Optional[torch.Tensor] = None,
                    new_k_rows: Optional[torch.Tensor] = None,
                    new_v_rows: Optional[torch.Tensor] = None,
                    partials: Optional[torch.Tensor] = None,
                    counters: Optional[torch.Tensor] = None, fused_merge: bool = False) -> None:
    """Varlen paged attention into ``out_rows`` ((rows, Hq, D) views, device).

    Split-K partitions are merged by a separate merge kernel; with
    ``fused_merge`` the attention kernel merges them itself (the last partition
    of a group to finish, through arrival counters from the workspace unless
    given) -- correct, but slower on MI355X because every arriving partition
    must release its partials with an agent-scope fence."""
    _rows_ok(q_rows, "q_rows")
    _rows_ok(out_rows, "out_rows")
    require_device(q_rows, out_rows, pool.k, block_tables, cu_seqlens, kv_lens, positions)
    if q_rows.dtype != pool.k.dtype or out_rows.dtype != pool.k.dtype:
        raise TypeError("query, output and pool must share a dtype")
    for name, t, dt in (("block_tables", block_tables, torch.int32), ("cu_seqlens", cu_seqlens, torch.int32),
                        ("kv_lens", kv_lens, torch.int32), ("positions", positions, torch.int64)):
        if t.dtype != dt or not t.is_contiguous():
            raise TypeError(f"{name} must be a contiguous {dt} tensor")
    Hq, D = q_rows.shape[1], q_rows.shape[2]
    if isinstance(plan, CountedPlan):
        return _paged_attention_counted(q_rows, out_rows, pool, block_tables, cu_seqlens, kv_lens, positions,
                                        plan, scale, num_kv_heads, row_map, pool_lens, new_k_rows, new_v_rows)
    if partials is None:
        partials = _WORKSPACE.partials(plan.partials_floats, q_rows.device)
    if plan.sliced:
        if row_map is not None or pool_lens is not None or fused_merge:
            raise ValueError("a slice plan takes no row map, in-flight keys or fused merge")
        bt_stride = block_tables.shape[1] if block_tables.dim() == 2 else 0
        _check(lib().mf_paged_attention_slices(
            _ptr(q_rows), q_rows.stride(0), q_rows.stride(1),
            _ptr(out_rows), out_rows.stride(0), out_rows.stride(1),
            dtype_code(q_rows.dtype), _ptr(pool.k), _ptr(pool.v),
            pool.stride_block, pool.stride_slot, pool.stride_head, pool.block_size,
            _ptr(block_tables), bt_stride, _ptr(cu_seqlens), _ptr(kv_lens), _ptr(positions),
            Hq, num_kv_heads, D, float(scale),
            _ptr(plan.items), plan.n_narrow, plan.n_wide, _ptr(plan.merges), plan.n_merges,
            _ptr(partials), partials.numel() if partials is not None else 0, _stream(q_rows.device),
        ), "mf_paged_attention_slices")
        return
    if fused_merge and counters is None:
        counters = _WORKSPACE.counters(plan.n_merges, q_rows.device)
    if not fused_merge:
        counters = None
    nk = new_k_rows if new_k_rows is not None else None
    nv = new_v_rows if new_v_rows is not None else None
    if pool_lens is not None:
        if nk is None or nv is None:
            raise ValueError("pool_lens needs the in-flight new_k_rows/new_v_rows")
        require_device(pool_lens, nk, nv)
        if not same_layout(nk, nv):
            raise ValueError("in-flight K and V rows must share strides")
    bt_stride = block_tables.shape[1] if block_tables.dim() == 2 else 0
    _check(lib().mf_paged_attention(
        _ptr(q_rows), q_rows.stride(0), q_rows.stride(1),
        _ptr(out_rows), out_rows.stride(0), out_rows.stride(1),
        dtype_code(q_rows.dtype), _ptr(pool.k), _ptr(pool.v),
        pool.stride_block, pool.stride_slot, pool.stride_head, pool.block_size,
        _ptr(block_tables), bt_stride, _ptr(cu_seqlens), _ptr(kv_lens), _ptr(positions),
        _ptr(row_map), _ptr(pool_lens), _ptr(nk), _ptr(nv),
        nk.stride(0) if nk is not None else 0, nk.stride(1) if nk is not None else 0,
        Hq, num_kv_heads, D, float(scale),
        _ptr(plan.items), plan.n_narrow, plan.n_wide, _ptr(plan.merges), plan.n_merges,
        _ptr(partials), partials.numel() if partials is not None else 0, _ptr(counters), _stream(q_rows.device),
    ), "mf_paged_attention")


def paged_attention_kv_write(q_rows: torch.Tensor, out_rows: torch.Tensor, pool: PoolView,
                             block_tables: torch.Tensor, cu_seqlens: torch.Tensor, kv_lens: torch.Tensor,
                             positions: torch.Tensor, plan, scale: float, num_kv_heads: int,
                             new_k_rows: torch.Tensor, new_v_rows: torch.Tensor,
                             slot_mapping: torch.Tensor) -> None:
    """One launch for a packed step's KV write and its attention
    (mf_paged_attention_kv_write): rows ``new_k_rows``/``new_v_rows``
    ((rows, Hkv, D) views in the pool's dtype) go to the pool through
    ``slot_mapping`` (int64; slot -1 skips a row), and every sequence's keys
    from ``kv_lens[s] - q_len[s]`` on are read from those rows instead of the
    pool. Row cu_seqlens[s] + i must be sequence s's new token at position
    kv_lens[s] - q_len[s] + i. ``plan`` is an AttentionPlan or a CountedPlan
    (graph capture). Same pool contents and output as ``kv_write`` followed by
    ``paged_attention``."""
    _rows_ok(q_rows, "q_rows")
    _rows_ok(out_rows, "out_rows")
    _rows_ok(new_k_rows, "new_k_rows")
    _rows_ok(new_v_rows, "new_v_rows")
    require_device(q_rows, out_rows, pool.k, block_tables, cu_seqlens, kv_lens, positions, new_k_rows,
                   new_v_rows, slot_mapping)
    if q_rows.dtype != pool.k.dtype or out_rows.dtype != pool.k.dtype or new_k_rows.dtype != pool.k.dtype \
            or new_v_rows.dtype != pool.k.dtype:
        raise TypeError("query, output, new rows and pool must share a dtype")
    if not same_layout(new_k_rows, new_v_rows):
        raise ValueError("new K and V rows must share shape and strides")
    if slot_mapping.dtype != torch.int64 or not slot_mapping.is_contiguous():
        raise TypeError("slot_mapping must be a contiguous int64 tensor")
    T, H, D = new_k_rows.shape
    if H != pool.num_heads or D != pool.head_dim or slot_mapping.numel() != T:
        raise ValueError(f"new rows {tuple(new_k_rows.shape)} / {slot_mapping.numel()} slots do not match a "
                         f"pool of {pool.num_heads} heads x {pool.head_dim}")
    if getattr(plan, "sliced", False):
        raise ValueError("a written-in-flight step takes per-range plans (mf_attention_plan)")
    bt_stride = block_tables.shape[1] if block_tables.dim() == 2 else 0
    if isinstance(plan, CountedPlan):
        n_narrow, n_wide, n_merges = plan.cap_narrow, plan.cap_wide, plan.cap_merges
        counts, partials = plan.counts, plan.partials
    else:
        n_narrow, n_wide, n_merges = plan.n_narrow, plan.n_wide, plan.n_merges
        counts, partials = None, _WORKSPACE.partials(plan.partials_floats, q_rows.device)
        # every item's rows (its sequence's first row and row count) must be
        # rows of the new K/V the launch reads in flight
        held = plan.items_host[: n_narrow + n_wide]
        if held.shape[0] and int((held[:, 8] + held[:, 9]).max()) > T:
            raise ValueError(f"the plan's sequences reach past the {T} new rows")
    _check(lib().mf_paged_attention_kv_write(
        _ptr(q_rows), q_rows.stride(0), q_rows.stride(1),
        _ptr(out_rows), out_rows.stride(0), out_rows.stride(1),
        dtype_code(q_rows.dtype), _ptr(pool.k), _ptr(pool.v),
        pool.stride_block, pool.stride_slot, pool.stride_head, pool.block_size,
        _ptr(block_tables), bt_stride, _ptr(cu_seqlens), _ptr(kv_lens), _ptr(positions),
        _ptr(new_k_rows), _ptr(new_v_rows), new_k_rows.stride(0), new_k_rows.stride(1),
        _ptr(slot_mapping), T, pool.num_slots,
        q_rows.shape[1], num_kv_heads, q_rows.shape[2], float(scale),
        _ptr(plan.items), n_narrow, n_wide, _ptr(plan.merges), n_merges, _ptr(counts),
        _ptr(partials), partials.numel() if partials is not None else 0, _stream(q_rows.device),
    ), "mf_paged_attention_kv_write")


# fp32 partials the no-allocation entry point holds per GPU (32 MiB)
NOALLOC_PARTIALS_FLOATS = 8 * 1024 * 1024


def plan_partials_reach(plan: AttentionPlan, head_dim: int) -> int:
    """fp32 partial floats up to the end of the highest partial slot a
    per-range plan's items or merge records name. The kernels take the slot
    numbers as given, so this (not a declared size) is what a buffer must
    hold."""
    stride = 16 * (max(32, head_dim) + 2)
    top = 0
    n_items = plan.n_narrow + plan.n_wide
    if n_items:
        it = np.asarray(plan.items_host[:n_items], dtype=np.int64)
        named = it[:, 6] >= 0
        if named.any():
            # an item writes slots pslot .. pslot + column tiles - 1
            top = max(top, int((it[named, 6] + np.maximum(it[named, 3], 1)).max()))
    if plan.n_merges:
        mg = np.asarray(plan.merges_host[:plan.n_merges], dtype=np.int64)
        # record: partitions mg[3] at slot mg[4] + p * mg[5]
        top = max(top, int((mg[:, 4] + (np.maximum(mg[:, 3], 1) - 1) * mg[:, 5] + 1).max()))
    return top * stride


def paged_attention_noalloc(q_rows: torch.Tensor, out_rows: torch.Tensor, pool: PoolView,
                            block_tables: torch.Tensor, cu_seqlens: torch.Tensor, kv_lens: torch.Tensor,
                            positions: torch.Tensor, plan: AttentionPlan, scale: float, num_kv_heads: int,
                            row_map: Optional[torch.Tensor] = None, pool_lens: Optional[torch.Tensor] = None,
                            new_k_rows: Optional[torch.Tensor] = None,
                            new_v_rows: Optional[torch.Tensor] = None) -> None:
    """``paged_attention`` through mf_paged_attention_noalloc: the split-K
    partials live in the library's own per-GPU array, so the call allocates
    nothing (neither here nor in the library). Plans needing more than
    NOALLOC_PARTIALS_FLOATS partial floats are refused."""
    if getattr(plan, "sliced", False):
        raise ValueError("the no-allocation entry point takes per-range plans (mf_attention_plan)")
    # The slots the plan's items and merge records name must lie inside the
    # library's array, whatever partials_floats declares: no kernel bounds a
    # slot against it.
    reach = max(plan_partials_reach(plan, q_rows.shape[2]), plan.partials_floats)
    if reach > NOALLOC_PARTIALS_FLOATS:
        raise MemforgeHipError(
            f"mf_paged_attention_noalloc: the plan's partial slots need {reach} floats, past the "
            f"{NOALLOC_PARTIALS_FLOATS} of the library's array (workspace too small)")
    _rows_ok(q_rows, "q_rows")
    _rows_ok(out_rows, "out_rows")
    require_device(q_rows, out_rows, pool.k, block_tables, cu_seqlens, kv_lens, positions)
    if q_rows.dtype != pool.k.dtype or out_rows.dtype != pool.k.dtype:
        raise TypeError("query, output and pool must share a dtype")
    nk, nv = new_k_rows, new_v_rows
    if pool_lens is not None:
        if nk is None or nv is None:
            raise ValueError("pool_lens needs the in-flight new_k_rows/new_v_rows")
        require_device(pool_lens, nk, nv)
        if not same_layout(nk, nv):
            raise ValueError("in-flight K and V rows must share strides")
    bt_stride = block_tables.shape[1] if block_tables.dim() == 2 else 0
    _check(lib().mf_paged_attention_noalloc(
        _ptr(q_rows), q_rows.stride(0), q_rows.stride(1),
        _ptr(out_rows), out_rows.stride(0), out_rows.stride(1),
        dtype_code(q_rows.dtype), _ptr(pool.k), _ptr(pool.v),
        pool.stride_block, pool.stride_slot, pool.stride_head, pool.block_size,
        _ptr(block_tables), bt_stride, _ptr(cu_seqlens), _ptr(kv_lens), _ptr(positions),
        _ptr(row_map), _ptr(pool_lens), _ptr(nk), _ptr(nv),
        nk.stride(0) if nk is not None else 0, nk.stride(1) if nk is not None else 0,
        q_rows.shape[1], num_kv_heads, q_rows.shape[2], float(scale),
        _ptr(plan.items), plan.n_narrow, plan.n_wide, _ptr(plan.merges), plan.n_merges,
        plan.partials_floats, _stream(q_rows.device),
    ), "mf_paged_attention_noalloc")


def paged_attention_packed(q_rows: torch.Tensor, out_rows: torch.Tensor, pool: PoolView, buf: torch.Tensor,
                           offsets: Sequence[int], num_seqs: int, bt_stride: int, counts: np.ndarray,
                           scale: float, num_kv_heads: int, has_row_map: bool, has_pool_lens: bool,
                           new_k_rows: Optional[torch.Tensor] = None,
                           new_v_rows: Optional[torch.Tensor] = None, sliced: bool = False) -> None:
    """mf_paged_attention on index arrays that one ``upload`` placed in the
    device buffer ``buf`` at ``offsets`` (int32 words, as ``_layout`` gives
    them): the padded block tables, the plan's items, its merges, cu_seqlens
    followed by kv_lens (``num_seqs`` + 1 and ``num_seqs`` int32), the int64
    positions, then the row map and the pool lengths when present. The caller
    built all of them, so only the tensors it did not build (query, output,
    pool, in-flight rows) are checked, and the launch takes addresses inside
    ``buf`` instead of building a tensor view per array. ``sliced``: the plan
    is a slice plan (mf_paged_attention_slices; no row map or pool lengths)."""
    _rows_ok(q_rows, "q_rows")
    _rows_ok(out_rows, "out_rows")
    require_device(q_rows, out_rows, pool.k, buf)
    if q_rows.dtype != pool.k.dtype or out_rows.dtype != pool.k.dtype:
        raise TypeError("query, output and pool must share a dtype")
    if buf.dtype != torch.int32 or not buf.is_contiguous():
        raise TypeError("buf must be a contiguous int32 tensor")
    nk, nv = new_k_rows, new_v_rows
    if has_pool_lens:
        if nk is None or nv is None:
            raise ValueError("pool_lens needs the in-flight new_k_rows/new_v_rows")
        require_device(nk, nv)
        if not same_layout(nk, nv):
            raise ValueError("in-flight K and V rows must share strides")
    dev = q_rows.device
    n_narrow, n_wide, n_merges, floats = (int(x) for x in counts)
    partials = _WORKSPACE.partials(floats, dev)
    addr = [buf.data_ptr() + 4 * o for o in offsets]
    if sliced:
        if has_row_map or has_pool_lens:
            raise ValueError("a slice plan takes no row map or in-flight keys")
        _check(lib().mf_paged_attention_slices(
            _ptr(q_rows), q_rows.stride(0), q_rows.stride(1),
            _ptr(out_rows), out_rows.stride(0), out_rows.stride(1),
            dtype_code(q_rows.dtype), _ptr(pool.k), _ptr(pool.v),
            pool.stride_block, pool.stride_slot, pool.stride_head, pool.block_size,
            addr[0], bt_stride, addr[3], addr[3] + 4 * (num_seqs + 1), addr[4],
            q_rows.shape[1], num_kv_heads, q_rows.shape[2], float(scale),
            addr[1], n_narrow, n_wide, addr[2], n_merges,
            _ptr(partials), partials.numel() if partials is not None else 0, _stream(dev),
        ), "mf_paged_attention_slices")
        return
    row_map = addr[5] if has_row_map else None
    pool_lens = addr[5 + int(has_row_map)] if has_pool_lens else None
    _check(lib().mf_paged_attention(
        _ptr(q_rows), q_rows.stride(0), q_rows.stride(1),
        _ptr(out_rows), out_rows.stride(0), out_rows.stride(1),
        dtype_code(q_rows.dtype), _ptr(pool.k), _ptr(pool.v),
        pool.stride_block, pool.stride_slot, pool.stride_head, pool.block_size,
        addr[0], bt_stride, addr[3], addr[3] + 4 * (num_seqs + 1), addr[4],
        row_map, pool_lens, _ptr(nk), _ptr(nv),
        nk.stride(0) if nk is not None else 0, nk.stride(1) if nk is not None else 0,
        q_rows.shape[1], num_kv_heads, q_rows.shape[2], float(scale),
        addr[1], n_narrow, n_wide, addr[2], n_merges,
        _ptr(partials), partials.numel() if partials is not None else 0, None, _stream(dev),
    ), "mf_paged_attention")


def _paged_attention_counted(q_rows, out_rows, pool, block_tables, cu_seqlens, kv_lens, positions,
                             plan: CountedPlan, scale, num_kv_heads, row_map, pool_lens, nk, nv) -> None:
    if pool_lens is not None:
        if nk is None or nv is None:
            raise ValueError("pool_lens needs the in-flight new_k_rows/new_v_rows")
        require_device(pool_lens, nk, nv)
    Hq, D = q_rows.shape[1], q_rows.shape[2]
    bt_stride = block_tables.shape[1] if block_tables.dim() == 2 else 0
    _check(lib().mf_paged_attention_counted(
        _ptr(q_rows), q_rows.stride(0), q_rows.stride(1),
        _ptr(out_rows), out_rows.stride(0), out_rows.stride(1),
        dtype_code(q_rows.dtype), _ptr(pool.k), _ptr(pool.v),
        pool.stride_block, pool.stride_slot, pool.stride_head, pool.block_size,
        _ptr(block_tables), bt_stride, _ptr(cu_seqlens), _ptr(kv_lens), _ptr(positions),
        _ptr(row_map), _ptr(pool_lens), _ptr(nk), _ptr(nv),
        nk.stride(0) if nk is not None else 0, nk.stride(1) if nk is not None else 0,
        Hq, num_kv_heads, D, float(scale),
        _ptr(plan.items), plan.cap_narrow, plan.cap_wide, _ptr(plan.merges), plan.cap_merges,
        _ptr(plan.counts), _ptr(plan.partials), plan.partials.numel(), _stream(q_rows.device),
    ), "mf_paged_attention_counted")


# -------------------------------------------------------------- ragged pack

@dataclass
class PackedStep:
    token_ids: torch.Tensor     # int64 [T]
    positions: torch.Tensor     # int64 [T]
    seq_slot: torch.Tensor      # int32 [T]
    slot_mapping: torch.Tensor  # int64 [T]
    cu_seqlens: torch.Tensor    # int32 [B+1]
    kv_lens: torch.Tensor       # int32 [B]
    block_tables: torch.Tensor  # int32 [B, max_blocks]
    status: torch.Tensor        # int32 [4]

    @classmethod
    def allocate(cls, total_tokens: int, num_entries: int, max_blocks: int, device) -> "PackedStep":
        return cls(
            token_ids=torch.empty(total_tokens, dtype=torch.int64, device=device),
            positions=torch.empty(total_tokens, dtype=torch.int64, device=device),
            seq_slot=torch.empty(total_tokens, dtype=torch.int32, device=device),
            slot_mapping=torch.empty(total_tokens, dtype=torch.int64, device=device),
            cu_seqlens=torch.empty(num_entries + 1, dtype=torch.int32, device=device),
            kv_lens=torch.empty(num_entries, dtype=torch.int32, device=device),
            block_tables=torch.empty((num_entries, max_blocks), dtype=torch.int32, device=device),
            status=torch.empty(4, dtype=torch.int32, device=device),
        )


def check_pack_entries(entries: np.ndarray, tables: np.ndarray, tokens_len: int, total_tokens: int,
                       num_blocks: Optional[int] = None) -> None:
    """Host check of ragged-pack descriptors before they go to the device:
    every field non-negative, every table run inside ``tables`` and every
    token run inside ``tokens_len``, the row count equal to the sum of q_len,
    and (with ``num_blocks``) every block id the runs name inside the pool.
    Raises ValueError / IndexError naming the first bad entry."""
    ent = np.asarray(entries, dtype=np.int64).reshape(-1, ENTRY_INTS)
    if ent.shape[0] == 0:
        if total_tokens:
            raise ValueError(f"{total_tokens} packed rows but no entries")
        return
    bad = np.flatnonzero((ent[:, [0, 2, 3, 4, 5]] < 0).any(axis=1)
                         | (ent[:, 3] + ent[:, 4] > len(tables))
                         | (ent[:, 5] + ent[:, 0] > tokens_len))
    if bad.size:
        e = int(bad[0])
        raise ValueError(f"ragged-pack entry {e} is malformed: {ent[e].tolist()} against "
                         f"{len(tables)} table ids and {tokens_len} tokens")
    rows = int(ent[:, 0].sum())
    if rows != total_tokens:
        raise ValueError(f"entries hold {rows} rows, the step declares {total_tokens}")
    if num_blocks is not None and len(tables):
        t = np.asarray(tables)
        lo, hi = int(t.min()), int(t.max())
        if lo < 0 or hi >= num_blocks:
            raise IndexError(f"block id {lo if lo < 0 else hi} is outside a pool of {num_blocks} blocks")


def ragged_pack(entries: torch.Tensor, tables: torch.Tensor, tokens: torch.Tensor,
                total_tokens: int, block_size: int, max_blocks: int,
                slot_bitmap: Optional[torch.Tensor] = None, num_slots: int = 0,
                out: Optional[PackedStep] = None) -> PackedStep:
    """Run mf_ragged_pack on device descriptors (int32 tensors already on the
    GPU), into ``out``'s buffers when given (they must be sized for
    ``total_tokens`` rows, ``entries.shape[0]`` entries and ``max_blocks``).
    The kernel bounds every load by ``tables.numel()`` / ``tokens.numel()``
    and, with ``num_slots``, every block id by the pool; host callers that
    built the descriptors check them first with ``check_pack_entries``."""
    require_device(entries, tables, tokens)
    if entries.dtype != torch.int32 or tables.dtype != torch.int32 or tokens.dtype != torch.int32:
        raise TypeError("ragged_pack takes int32 entries, tables and tokens")
    if not (entries.is_contiguous() and tables.is_contiguous() and tokens.is_contiguous()):
        raise ValueError("ragged_pack takes contiguous entries, tables and tokens")
    dev = entries.device
    B = entries.shape[0]
    if out is not None:
        if (out.token_ids.numel() != total_tokens or out.cu_seqlens.numel() != B + 1
                or tuple(out.block_tables.shape) != (B, max_blocks)):
            raise ValueError("preallocated pack buffers do not match the step")
    else:
        out = PackedStep.allocate(total_tokens, B, max_blocks, dev)
    _check(lib().mf_ragged_pack(
        _ptr(entries), B, _ptr(tables), tables.numel(), _ptr(tokens), tokens.numel(), block_size,
        max_blocks, total_tokens,
        _ptr(out.token_ids), _ptr(out.positions), _ptr(out.seq_slot), _ptr(out.slot_mapping),
        _ptr(out.cu_seqlens), _ptr(out.kv_lens), _ptr(out.block_tables), _ptr(slot_bitmap),
        num_slots, _ptr(out.status), _stream(),
    ), "mf_ragged_pack")
    return out


# --------------------------------------------------------- rejection verify

@dataclass
class VerifyResult:
    tokens: torch.Tensor        # int32 [B, K+1]
    is_draft: torch.Tensor      # uint8 [B, K+1]
    count: torch.Tensor         # int32 [B]
    num_accepted: torch.Tensor  # int32 [B]


_VERIFY_WS_BYTES = {}  # (rows, candidates) -> mf_spec_verify_workspace_size


def spec_verify(draft_tokens: torch.Tensor, draft_probs: torch.Tensor, target_logits: torch.Tensor,
                temperature: float, u_accept: torch.Tensor, exp_noise: torch.Tensor,
                target_is_probs: bool = False) -> VerifyResult:
    """Batched rejection sampling. Shapes: draft_tokens (B, K) int32,
    draft_probs (B, K, V) fp32, target_logits (B, K+1, >=V) -- or target
    probabilities (fp32) with ``target_is_probs`` --, u_accept (B, K) fp32,
    exp_noise (B, V) fp32."""
    require_device(draft_tokens, draft_probs, target_logits, u_accept, exp_noise)
    B, K = draft_tokens.shape
    V = draft_probs.shape[-1] if K > 0 else exp_noise.shape[-1]
    if target_logits.shape[0] != B or target_logits.shape[1] != K + 1 or target_logits.shape[2] < V:
        raise ValueError(f"target logits {tuple(target_logits.shape)} do not cover ({B}, {K + 1}, {V})")
    if target_logits.stride(-1) != 1 or draft_probs.stride(-1) != 1 or exp_noise.stride(-1) != 1:
        raise ValueError("vocabulary axes must be contiguous")
    if draft_tokens.dtype != torch.int32 or not draft_tokens.is_contiguous():
        draft_tokens = draft_tokens.to(torch.int32).contiguous()
    if u_accept.dtype != torch.float32 or not u_accept.is_contiguous():
        u_accept = u_accept.to(torch.float32).contiguous()
    dev = target_logits.device
    # one allocation for the four outputs (only the first count[b] entries of
    # each row are written); is_draft is bytes of its int32 tail. The kernels
    # are queued first and the views built after, so no view is made on the
    # way to the launch.
    n = B * (K + 1)
    out = torch.empty(n + 2 * B + (n + 3) // 4, dtype=torch.int32, device=dev)
    base = out.data_ptr()
    L = lib()
    ws_bytes = _VERIFY_WS_BYTES.get((B, K))
    if ws_bytes is None:
        ws_bytes = _VERIFY_WS_BYTES[(B, K)] = int(L.mf_spec_verify_workspace_size(B, K))
    stream = _stream(dev)
    ws = _WORKSPACE.verify(ws_bytes, dev, stream)
    _check(L.mf_spec_verify(
        B, K, V, draft_tokens.data_ptr(), draft_probs.data_ptr(),
        draft_probs.stride(0) if K > 0 else 0, draft_probs.stride(1) if K > 0 else 0,
        target_logits.data_ptr(), dtype_code(target_logits.dtype), target_logits.stride(0),
        target_logits.stride(1), float(temperature), int(bool(target_is_probs)), u_accept.data_ptr(),
        exp_noise.data_ptr(), exp_noise.stride(0), base, base + 4 * (n + 2 * B), base + 4 * n,
        base + 4 * (n + B), ws.data_ptr(), ws_bytes, stream,
    ), "mf_spec_verify")
    return VerifyResult(
        tokens=out[:n].view(B, K + 1),
        is_draft=out[n + 2 * B:].view(torch.uint8)[:n].view(B, K + 1),
        count=out[n:n + B],
        num_accepted=out[n + B:n + 2 * B],
    )
