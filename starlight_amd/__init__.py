"""starlight_amd — MI355X (gfx950) compute backend for StarLight.

The product is the C-ABI library `lib/libstarlight_hip.so` (sources in
`csrc/`, interface in `include/starlight_hip.h`) implementing the
`sl_device::Device` contract. This package is its host-side mirror:
`ir` (sl-ir types), `device` (the Device trait over the C ABI), `quant`
(the group-wise quantization convention), `graph`/`engine` (the thin slice of
sl-graph / sl-model-adapters / sl-core that drives it).
"""
from . import ir  # noqa: F401
