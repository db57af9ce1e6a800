"""q36_amd: MI355X-native W4A8 mixture-of-experts layer for the q36 engine.

The compute path is libq36moe.so (HIP, gfx950), reached through the C ABI in
include/q36moe.h.  `q36_amd.moe` is the Python host mirror over that ABI;
`q36_amd.synth` builds seeded synthetic inputs.
"""
from . import synth  # noqa: F401

__all__ = ["synth", "moe"]
