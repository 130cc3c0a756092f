"""sushi_amd: MI355X-native (gfx950, HIP) EXL3/STQ trellis-quantized linear hot path of beamivalice/sushi.

``sushi_amd.exl3`` mirrors the reference's ``sushi_exl3`` operator API over the C ABI in
``include/sushi_exl3_hip.h``; ``sushi_amd.pack`` loads EXL3/STQ packs (safetensors shards) into device banks;
``sushi_amd.synth`` builds seeded synthetic banks; ``sushi_amd.build`` compiles the HIP library in-tree.
"""
from . import exl3, pack, synth  # noqa: F401

__all__ = ["exl3", "pack", "synth"]
