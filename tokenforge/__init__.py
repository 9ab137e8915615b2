"""TokenForge's quantized-linear path on MI355X (gfx950).

``tokenforge.kernels`` is the drop-in host side of the reference's package of the same name;
its compute runs in the HIP kernel library built from ``tokenforge_amd/csrc``.
"""
