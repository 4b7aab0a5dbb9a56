"""fathom_amd: MI355X (gfx950) implementation of Fathom's bit-plane key-scan path.

``fathom_amd.bitplane`` is the drop-in for the reference module
kernels/bitplane.py; ``fathom_amd.offload`` holds the host-resident store
helpers and the top-k row gather.  All compute runs in libfathom_hip.so.
"""
__version__ = "0.1.0"
