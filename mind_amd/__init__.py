"""MI355X-native edge-set attention (ESA) hot path of HUBioDataLab/MIND.

Hand-written gfx950 HIP kernels behind the C ABI in ``include/esa_hip.h``
(``mind_amd/lib/libesa_hip.so``), with PyTorch modules that keep the
reference's ``esa/mha.py`` and ``esa/mha_flash_varlen.py`` signatures.
"""
__version__ = "0.1.0"
