"""Small numpy helpers for building test inputs."""
import numpy as np


def rb(x) -> np.ndarray:
    """round_bf16 (src/tensor.rs:645-652) vectorised, for building inputs."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    r = np.where(nan, ((b & 0xFFFF0000) | 0x00400000).astype(np.uint32), r)
    return r.view(np.float32)


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


_mapping = [1000]


def fresh_mapping() -> int:
    """A new `mapping` id for yue2_hip_vector/ar_stack weights: the device
    weight cache is keyed by (mapping, address, shape, dtype), and the
    mapping id is what keeps a reused host address from aliasing."""
    _mapping[0] += 1
    return _mapping[0]
