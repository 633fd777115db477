"""Measured figures of a running engine: device memory and data-path bandwidth.

The reference reports where its pool lives and what the device holds
(memforge_ml/runtime/continuous_engine.py:1432-1483); a dashboard reads those
keys, so they keep their names. On top, ``DataPathMeter`` measures the
bandwidth the data-path kernels reach inside the engine, without a profiler:

* every ``every``-th forward pass is sampled;
* on a sampled eager pass, one layer's KV write and attention launch (or
  the one launch doing both, family ``attention_kv_write``) are timed with
  HIP events on the stream the kernels run on. An eager pass is
  usually host-bound -- the GPU waits for each launch -- so an event recorded
  just before a launch would time the host's enqueue latency too. The timed
  launch is therefore preceded by a short GPU spin (about 40 us, recalibrated
  from each sample): the start event is recorded after the spin, by which
  time the launch is already queued behind it, so start-to-end is the
  kernel's own time;
* on a sampled graph replay (a captured decode step) the events bracket the
  replay itself; its bytes are the step's: every weight once, plus every
  layer's attention and KV-write bytes (the decode step's bytes roofline);
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
_SPIN_TARGET_US = 40.0


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


def _event() -> torch.cuda.Event:
    ev = torch.cuda.Event(enable_timing=True)
    ev.record()
    return ev


class _PassRecord:
    """The events of one sampled pass: per kernel family a list of
    (spin start, kernel start, kernel end) events; the spin start is None
    where nothing precedes the timed work."""

    __slots__ = ("bytes", "layer", "spin_cycles", "events")

    def __init__(self, nbytes: Dict[str, int], layer: Optional[int], spin_cycles: int):
        self.bytes = nbytes
        self.layer = layer
        self.spin_cycles = spin_cycles
        self.events: Dict[str, List[Tuple[Optional[torch.cuda.Event], torch.cuda.Event, torch.cuda.Event]]] = {}

    def start(self, layer: Optional[int] = None):
        """Before a launch of layer ``layer``: spin, then the start event (only
        for the record's timed layer; None for every other layer)."""
        if layer != self.layer:
            return None
        spin = _event()
        torch.cuda._sleep(self.spin_cycles)
        return spin, _event()

    def stop(self, family: str, began) -> None:
        if began is not None:
            self.events.setdefault(family, []).append((began[0], began[1], _event()))

    def start_whole(self):
        """Before a whole graph replay (no spin: one launch, no host gap)."""
        return None, _event()

    def done(self) -> bool:
        return all(e.query() for trips in self.events.values() for _, _, e in trips)


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
        self.timed_layer = spec.num_layers // 2
        self.spin_cycles = 100_000
        self._passes = 0
        self._pending: Deque[_PassRecord] = deque()
        # per family: [samples, bytes, seconds, last bytes per launch, last us per launch]
        self._totals: Dict[str, List[float]] = {}

    def arm(self) -> bool:
        """Whether the coming pass is a sampled one."""
        self._passes += 1
        return self.every > 0 and (self._passes - 1) % self.every == 0

    def layer_bytes(self, kv_lens: List[int], rows: int) -> Dict[str, int]:
        """Algorithmic bytes of one layer's attention and KV write."""
        kv = sum(int(n) for n in kv_lens)
        tables = sum((int(n) + self.block_size - 1) // self.block_size for n in kv_lens) * 4
        attention = 2 * kv * self.kv_row + tables + 2 * rows * self.q_row
        kv_write = 2 * 2 * rows * self.kv_row + 8 * rows
        return {"attention": attention, "kv_write": kv_write, "attention_kv_write": attention + kv_write}

    def step_bytes(self, kv_lens: List[int], rows: int) -> int:
        """Bytes roofline of a whole pass: weights once, every layer's data path."""
        per_layer = self.layer_bytes(kv_lens, rows)
        return self.weight_bytes + self.num_layers * (per_layer["attention"] + per_layer["kv_write"])

    def begin(self, nbytes: Dict[str, int], whole: bool = False) -> _PassRecord:
        """A record for one sampled pass: one timed layer of an eager pass, or
        (``whole``) a graph replay."""
        rec = _PassRecord(nbytes, None if whole else self.timed_layer, self.spin_cycles)
        self._pending.append(rec)
        return rec

    def poll(self) -> None:
        """Fold the completed records into the totals (never waits)."""
        while self._pending and self._pending[0].done():
            rec = self._pending.popleft()
            for family, trips in rec.events.items():
                secs = sum(b.elapsed_time(e) for _, b, e in trips) / 1e3
                spins = [s.elapsed_time(b) * 1e3 for s, b, _ in trips if s is not None]
                if spins:  # keep the spin near its target as clocks change
                    mean = sum(spins) / len(spins)
                    if mean > 0:
                        scaled = self.spin_cycles * _SPIN_TARGET_US / mean
                        self.spin_cycles = int(min(max(scaled, 10_000), 2_000_000))
                nbytes = rec.bytes.get(family, 0)
                t = self._totals.setdefault(family, [0, 0, 0.0, 0, 0.0])
                t[0] += 1
                t[1] += nbytes * len(trips)
                t[2] += secs
                t[3] = nbytes
                t[4] = secs / len(trips) * 1e6

    def snapshot(self) -> Dict[str, Any]:
        """The measured figures, one group of keys per kernel family."""
        self.poll()
        out: Dict[str, Any] = {"data_path_sample_every": self.every, "hbm_peak_gbps": HBM_PEAK_GBPS}
        for family in ("attention", "kv_write", "attention_kv_write", "decode_graph"):
            t = self._totals.get(family)
            if t is None or t[2] <= 0:
                out.update({f"{family}_samples": 0, f"{family}_gbps": None, f"{family}_hbm_frac": None,
                            f"{family}_us_per_launch": None, f"{family}_bytes_per_launch": None})
                continue
            gbps = t[1] / t[2] / 1e9
            out.update({
                f"{family}_samples": int(t[0]),
                f"{family}_gbps": round(gbps, 1),
                f"{family}_hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
                f"{family}_us_per_launch": round(t[4], 2),
                f"{family}_bytes_per_launch": int(t[3]),
            })
        return out
