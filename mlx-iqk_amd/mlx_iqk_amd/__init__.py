"""IQ_K routed-expert kernels for MI355X (gfx950), PyTorch-ROCm host side.

Modules, in dependency order:

- :mod:`mlx_iqk_amd.iq1grid` -- the IQ1_S ternary grid (shared with the C++/HIP code);
- :mod:`mlx_iqk_amd.format` -- the relayout definition, pack/unpack, reference decode;
- :mod:`mlx_iqk_amd.codec` -- the C++ quantizers and CPU dequantizers;
- :mod:`mlx_iqk_amd.kernels` -- guards and launch wrappers over ``libiqk_hip.so``;
- :mod:`mlx_iqk_amd.nn` -- :class:`IqkSwitchLinear`, the drop-in switch module;
- :mod:`mlx_iqk_amd.synth` -- seeded synthetic expert stacks for the routed geometry.
"""

from .format import MEMBERS, bits_per_weight, component_shapes, decode, pack, unpack

__all__ = ["MEMBERS", "IqkSwitchLinear", "bits_per_weight", "component_shapes", "decode", "pack", "unpack"]


def __getattr__(name):
    # torch is imported lazily so the format/codec layers work without it.
    if name == "IqkSwitchLinear":
        from .nn import IqkSwitchLinear
        return IqkSwitchLinear
    raise AttributeError(name)
