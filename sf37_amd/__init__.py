"""sf37_amd: MI355X (gfx950) implementation of the SF37 MoE feed-forward hot
path behind the C ABI in include/sf37_hip.h (libsf37_hip.so).

The HIP library is the product; this package only binds it (hip.py) and
builds seeded synthetic layers on the device (moe.py).
"""
from . import hip  # noqa: F401
