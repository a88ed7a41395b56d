"""Seeded synthetic workloads A-E of the benchmark (configs listed in BASELINE.json).

Shared settings: 4 branches, excitatory fraction 0.8, blocks of 256 neurons,
the reference's configs/test.toml dynamics and learning, context
{max_order 6, dim 16, slots 4096, probe 4, lr 0.02, confidence 8, dropout 0.5},
replay {fraction 0.30, segment 32, classic}, plasticity_window 1, seed 1337.
"Byte embedding 256xE" is Leo's input_fanout (context.embedding_dim is capped
at 256 by config.rs:447-451). Stories are Zipf(1.1)-ASCII text with a '\\n'
terminator, seed 0xC0FFEE ^ config index.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Tuple

import numpy as np

from . import native
from .config import Config, test_toml_values
from .model import Model


@dataclass(frozen=True)
class Workload:
    name: str
    index: int
    neurons: int
    synapses: int
    fanout: int
    lanes: int
    target_activity: float
    per_block: int
    global_cap: int
    stories: int
    length_mean: float
    length_std: float       # < 0: uniform in [min, max]
    length_min: int
    length_max: int
    topology: int
    exponent: float = 0.0
    in_degree_cap: int = 0
    eligibility_decay: float = 0.95


WORKLOADS: Dict[str, Workload] = {
    "A": Workload("A", 0, 1_024, 16, 64, 1, 0.02, 8, 32, 64, 0.0, -1.0, 256, 1024, native.TOPOLOGY_UNIFORM),
    "B": Workload("B", 1, 16_384, 32, 128, 8, 0.02, 8, 512, 4096, 800.0, 250.0, 64, 4096, native.TOPOLOGY_UNIFORM,
                  eligibility_decay=0.9),
    "C": Workload("C", 2, 131_072, 64, 256, 32, 0.05, 16, 8192, 50_000, 800.0, 250.0, 64, 4096,
                  native.TOPOLOGY_POWER_LAW, exponent=2.1),
    "D": Workload("D", 3, 1_048_576, 64, 512, 64, 0.01, 4, 16_384, 200_000, 800.0, 250.0, 64, 4096,
                  native.TOPOLOGY_UNIFORM),
    "E": Workload("E", 4, 4_194_304, 32, 256, 128, 0.30, 80, 1_310_720, 200_000, 3000.0, 1000.0, 64, 16_384,
                  native.TOPOLOGY_HEAVY_TAIL, exponent=1.1, in_degree_cap=4096),
}


def workload_config(w: Workload) -> Config:
    values = test_toml_values()
    values["model"].update(name=f"Leo-synthetic-{w.name}", seed=1337, neuron_count=w.neurons,
                           block_count=w.neurons // 256, neurons_per_block=256, synapses_per_neuron=w.synapses,
                           input_fanout=w.fanout, max_active_per_block=w.per_block, max_active_global=w.global_cap)
    values["dynamics"].update(target_activity=w.target_activity)
    values["learning"].update(eligibility_decay=w.eligibility_decay, plasticity_window=1)
    values["context"].update(max_order=6, embedding_dim=16, slots_per_order=4096, probe_limit=4, learning_rate=0.02,
                             confidence_observations=8, dropout_rate=0.5)
    values["replay"].update(fraction=0.30, segment_bytes=32, stateful_batch=False)
    return Config.from_dict(values)


def workload_model(w: Workload) -> Model:
    return Model.synthetic(workload_config(w), topology=w.topology, exponent=w.exponent,
                           in_degree_cap=w.in_degree_cap, weight_sigma=0.05)


def synthetic_stories(w: Workload, count: int, offset: int = 0) -> Tuple[np.ndarray, np.ndarray]:
    """The first offset+count stories of workload w; returns stories [offset, offset+count) packed."""
    lib = native.load()
    total = offset + count
    capacity = total * w.length_max + 16
    data = np.zeros(capacity, dtype=np.uint8)
    offsets = np.zeros(total + 1, dtype=np.uint64)
    native.check(lib, lib.leo_synthetic_stories(0xC0FFEE ^ w.index, total, w.length_mean, w.length_std, w.length_min,
                                                 w.length_max, data.ctypes.data, capacity, offsets.ctypes.data))
    start, end = int(offsets[offset]), int(offsets[total])
    return data[start:end].copy(), (offsets[offset:] - offsets[offset]).astype(np.uint64)


def story_list(data: np.ndarray, offsets: np.ndarray) -> List[bytes]:
    return [data[int(offsets[i]):int(offsets[i + 1])].tobytes() for i in range(len(offsets) - 1)]
