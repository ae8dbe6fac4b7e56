"""unifiedkv_amd - MI355X (gfx950) Page16 hot path of BP-KV.

Drop-in modules: ``unifiedkv_amd.page16_native`` (core/page16_native.py) and,
for flat ``import page16_native`` by the unchanged reference scheduler,
``unifiedkv_amd/dropin/``. Kernels live in libukv.so (C ABI: include/ukv.h).
"""
__version__ = "0.1.0"
