"""Host launchers of the gfx950 kernels (the counterparts of ``tokenforge.kernels.triton``).

Each launcher checks its inputs with the reference's exception types and messages,
allocates outputs with the torch caching allocator and launches on torch's current stream
through the C ABI. None of them synchronizes or reads tensor values on the host, except the
load-time range check of :func:`tokenforge.kernels.hip.layout.pack_int4`.
"""
