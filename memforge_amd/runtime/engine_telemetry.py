"""Measured figures of a running engine: device memory and data-path bandwidth.

The reference reports where its pool lives and what the device holds
(memforge_ml/runtime/continuous_engine.py:1432-1483); a dashboard reads those
keys, so they keep their names. On top, ``DataPathMeter`` measures the
bandwidth the data-path kernels reach inside the engine, without a profiler:

* every ``every``-th forward pass is sampled;
* on a sampled eager pass, HIP events bracket each layer's KV write and
  attention launch on the stream those kernels run on; on a sampled graph
  replay (a captured decode step) they bracket the whole replay, whose bytes
  are then the step's: every weight once, plus every layer's attention and
  KV-write bytes (the decode step's bytes roofline);
* events are read back only once they have completed (``Event.query``), so
  sampling never makes the host wait for the GPU;
* the bytes are algorithmic: attention reads every visible K and V row once,
  the block-table entries and the queries, and writes the output; the KV
  write reads each new row, writes it into the pool and reads its 8-byte slot.

Achieved GB/s is bytes over measured time; the fraction is against the
MI355X's 8 TB/s HBM peak.
"""

from __future__ import annotations

from collections import deque
from typing import Any, Deque, Dict, List, Optional, Tuple

import torch

HBM_PEAK_GBPS = 8000.0


def device_figures(pool) -> Dict[str, Any]:
    """Pool geometry and the device's memory, under the reference's keys."""
    mb = float(1 << 20)
    desc = pool.describe()
    free_b, total_b = torch.cuda.mem_get_info()
    return {
        "device": desc["device"],
        "dtype": desc["dtype"],
        "num_blocks": desc["num_blocks"],
        "block_size": desc["block_size"],
        "capacity_tokens": desc["capacity_tokens"],
        "pool_mb": desc["total_mb"],
        "cuda_available": True,
        "device_name": torch.cuda.get_device_name(torch.device(desc["device"])),
        "allocated_mb": round(torch.cuda.memory_allocated() / mb, 2),
        "peak_memory_mb": round(torch.cuda.max_memory_allocated() / mb, 2),
        "reserved_mb": round(torch.cuda.memory_reserved() / mb, 2),
        "vram_total_mb": round(total_b / mb, 2),
        "vram_free_mb": round(free_b / mb, 2),
    }


class _PassRecord:
    """The events of one sampled pass, grouped by kernel family."""

    __slots__ = ("kind", "bytes", "events")

    def __init__(self, kind: str, nbytes: Dict[str, int]):
        self.kind = kind
        self.bytes = nbytes
        self.events: Dict[str, List[Tuple[torch.cuda.Event, torch.cuda.Event]]] = {}

    def start(self) -> torch.cuda.Event:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        return ev

    def stop(self, family: str, begin: torch.cuda.Event) -> None:
        end = torch.cuda.Event(enable_timing=True)
        end.record()
        self.events.setdefault(family, []).append((begin, end))

    def done(self) -> bool:
        return all(e.query() for pairs in self.events.values() for _, e in pairs)


class DataPathMeter:
    """Sampled HIP-event timing of the attention and KV-write kernels."""

    def __init__(self, spec, num_q_heads: int, block_size: int, weight_bytes: int, every: int = 16):
        self.every = max(0, int(every))
        self.weight_bytes = int(weight_bytes)
        self.elt = torch.tensor([], dtype=spec.dtype).element_size()
        self.kv_row = spec.num_kv_heads * spec.head_dim * self.elt  # one token's K (or V) in one layer
        self.q_row = num_q_heads * spec.head_dim * self.elt
        self.block_size = block_size
        self.num_layers = spec.num_layers
        self._passes = 0
        self._pending: Deque[_PassRecord] = deque()
        # per family: [samples, launches, bytes, seconds, last bytes per launch, last us per launch]
        self._totals: Dict[str, List[float]] = {}

    def arm(self) -> bool:
        """Whether the coming pass is a sampled one."""
        self._passes += 1
        return self.every > 0 and self._passes % self.every == 1 % self.every

    def layer_bytes(self, kv_lens: List[int], rows: int) -> Dict[str, int]:
        """Algorithmic bytes of one layer's attention and KV write."""
        kv = sum(int(n) for n in kv_lens)
        tables = sum((int(n) + self.block_size - 1) // self.block_size for n in kv_lens) * 4
        return {"attention": 2 * kv * self.kv_row + tables + 2 * rows * self.q_row,
                "kv_write": 2 * 2 * rows * self.kv_row + 8 * rows}

    def step_bytes(self, kv_lens: List[int], rows: int) -> int:
        """Bytes roofline of a whole pass: weights once, every layer's data path."""
        per_layer = self.layer_bytes(kv_lens, rows)
        return self.weight_bytes + self.num_layers * (per_layer["attention"] + per_layer["kv_write"])

    def begin(self, kind: str, nbytes: Dict[str, int]) -> _PassRecord:
        rec = _PassRecord(kind, nbytes)
        self._pending.append(rec)
        return rec

    def poll(self) -> None:
        """Fold the completed records into the totals (never waits)."""
        while self._pending and self._pending[0].done():
            rec = self._pending.popleft()
            for family, pairs in rec.events.items():
                secs = sum(a.elapsed_time(b) for a, b in pairs) / 1e3
                nbytes = rec.bytes.get(family, 0)
                t = self._totals.setdefault(family, [0, 0, 0, 0.0, 0, 0.0])
                t[0] += 1
                t[1] += len(pairs)
                t[2] += nbytes * len(pairs)
                t[3] += secs
                t[4] = nbytes
                t[5] = secs / len(pairs) * 1e6

    def snapshot(self) -> Dict[str, Any]:
        """The measured figures, one group of keys per kernel family."""
        self.poll()
        out: Dict[str, Any] = {"data_path_sample_every": self.every, "hbm_peak_gbps": HBM_PEAK_GBPS}
        for family in ("attention", "kv_write", "decode_graph"):
            t = self._totals.get(family)
            if t is None or t[3] <= 0:
                out.update({f"{family}_samples": 0, f"{family}_gbps": None, f"{family}_hbm_frac": None,
                            f"{family}_us_per_launch": None, f"{family}_bytes_per_launch": None})
                continue
            gbps = t[2] / t[3] / 1e9
            out.update({
                f"{family}_samples": int(t[0]),
                f"{family}_gbps": round(gbps, 1),
                f"{family}_hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
                f"{family}_us_per_launch": round(t[5], 2),
                f"{family}_bytes_per_launch": int(t[4]),
            })
        return out
