"""MI355X-native (gfx950) NSN packed-KV path: codec, packed cache and fused dequant-attention readout.

Importing the package registers the ``torch.ops.nsn.*`` operators (``nsn_amd.ops``)."""
from . import ops  # noqa: F401  (registers torch.ops.nsn.*)
