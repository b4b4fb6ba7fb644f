"""MI355X (gfx950) shard-commitment path of zkIE: Goldilocks LDE, Poseidon2
Merkle commitment with openings, and the WHIR/FRI row fold, behind the C ABI
of libzkie_hip.so (include/zkie_hip.h)."""
from ._native import DeviceBuffer, ZkieError, load  # noqa: F401

__all__ = ["DeviceBuffer", "ZkieError", "load"]
