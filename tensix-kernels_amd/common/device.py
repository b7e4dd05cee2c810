"""Device-side helpers: the data types, the device handle, HBM "banks" and the width-sharding of weights.

The reference's device helpers (common/device.py of XylolabsInc/tensix-kernels) describe a Tensix chip: DRAM banks,
core grids, NoC virtual channels, L1. On MI355X the HBM channel interleave is done by the hardware, so what survives
is the part with an observable effect on the API:

- `dram_banks` / `MAX_BANKS` / `check_banks` (reference common/device.py:29, 37-42, 56-62): a weight remembers how many
  banks it was "sharded" over and a matmul refuses a weight over more banks than `max_banks` with ValueError;
- `sharded_memcfg` (reference common/device.py:65-71): N padded to a multiple of banks * 32;
- the data types (the reference's ttnn.bfloat8_b, ttnn.bfloat4_b, ttnn.bfloat16, ttnn.float32, ttnn.uint32).

Placement, read VCs, split-loader arguments and L1 budgets have no MI355X meaning and are absent.
"""

import enum
import math
from dataclasses import dataclass

import torch

TILE = 32

# MI355X: eight HBM3E stacks; a weight's "banks" are the number it was padded for (N to banks * 32)
HBM_STACKS = 8
# Caps the banks a weight is sharded over (None: every bank the device reports)
MAX_BANKS = None
# MI355X compute units (the grid matmul's records default to; see dense_reader.linear.topk_result)
CU_GRID = (16, 16)

FIDELITY = ("lofi", "hifi2", "hifi3", "hifi4")  # accepted names; the MI355X path always accumulates in fp32


class DataType(enum.Enum):
    bfloat8_b = 0
    bfloat4_b = 1
    bfloat16 = 2
    float32 = 3
    uint32 = 4


bfloat8_b = DataType.bfloat8_b
bfloat4_b = DataType.bfloat4_b
bfloat16 = DataType.bfloat16
float32 = DataType.float32
uint32 = DataType.uint32

# the C ABI's format numbers (include/dense_reader.h)
FMT = {DataType.bfloat8_b: 0, DataType.bfloat4_b: 1, DataType.bfloat16: 2}


def as_dtype(d):
    """A DataType from a DataType, its name, or torch.bfloat16 / torch.float32."""
    if isinstance(d, DataType):
        return d
    if d is torch.bfloat16:
        return DataType.bfloat16
    if d is torch.float32:
        return DataType.float32
    if isinstance(d, str):
        return DataType[{"bfp8": "bfloat8_b", "bfp4": "bfloat4_b", "bf16": "bfloat16", "fp32": "float32"}.get(d, d)]
    raise TypeError(f"not a data type: {d!r}")


@dataclass(frozen=True)
class CoreCoord:
    x: int
    y: int


class Device:
    """One GPU: the torch device plus what the reference's device object answers that matters here."""

    def __init__(self, device_id=0):
        self.id = device_id
        self.torch = torch.device("cuda", device_id)

    def dram_grid_size(self):
        return CoreCoord(HBM_STACKS, 1)

    def compute_with_storage_grid_size(self):
        return CoreCoord(*CU_GRID)

    def stream(self):
        """The current HIP stream of this device (what the C ABI takes)."""
        return torch.cuda.current_stream(self.torch).cuda_stream

    def __repr__(self):
        return f"Device({self.id})"


def open_device(device_id=0):
    return Device(device_id)


def close_device(device):
    torch.cuda.synchronize(device.torch)


def as_device(device):
    """A Device from a Device, a torch.device, an int or None (cuda:0)."""
    if isinstance(device, Device):
        return device
    if device is None:
        return Device(0)
    if isinstance(device, int):
        return Device(device)
    d = torch.device(device)
    return Device(d.index or 0)


def dram_banks(device, max_banks=None):
    """The banks weights are sharded over: the device's, at most max_banks (default MAX_BANKS)."""
    n = as_device(device).dram_grid_size().x
    cap = max_banks if max_banks is not None else MAX_BANKS
    return min(n, cap) if cap else n


@dataclass(frozen=True)
class MemoryConfig:
    """Where a weight lives: width-sharded over `banks` (N padded to banks * 32) or interleaved (banks 0)."""

    banks: int
    shard_width: int = 0

    @property
    def sharded(self):
        return self.banks > 0


def sharded_memcfg(device, k, n, banks=None, max_banks=None):
    """Width-sharded over banks (default: dram_banks), N padded to a multiple of banks * 32."""
    banks = banks or dram_banks(device, max_banks)
    padded = math.ceil(n / (TILE * banks)) * TILE * banks
    return MemoryConfig(banks, padded // banks)


DRAM_MEMORY_CONFIG = MemoryConfig(0)
L1_MEMORY_CONFIG = MemoryConfig(0)


def is_dram_sharded(t):
    mc = getattr(t, "memory_config", None)
    return mc is not None and mc().sharded


def check_banks(t, max_banks=None):
    """ValueError for a weight sharded over more banks than max_banks (default MAX_BANKS; None: no limit)."""
    cap = max_banks if max_banks is not None else MAX_BANKS
    if t is not None and cap and is_dram_sharded(t) and t.memory_config().banks > cap:
        raise ValueError(f"a weight sharded over {t.memory_config().banks} DRAM banks (at most {cap}: max_banks)")
