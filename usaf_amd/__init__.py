"""usaf_amd -- MI355X-native (gfx950) quantized-expert hot path of USAF.

Hand-written HIP kernels (``csrc/``, built into ``libusaf_hip.so``, C-ABI in
``include/usaf_hip.h``) behind Python modules that keep the reference's call
sites: ``quantization`` (4-bit codec), ``qwen3moe_dml`` (routed expert
forward/backward), ``moe_loader`` (HBM-resident expert cache, sparse gradient
stores), ``sparse_optim`` (SparseAdam), ``cache`` / ``frozen_cache``.
"""
__version__ = "0.1.0"
