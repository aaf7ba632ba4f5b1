"""MI355X-native (gfx950) speculative-decoding verify step for nanoengine.

Hand-written HIP kernels (``csrc/``) behind the C ABI of ``libnanoengine_hip.so``
(``include/nanoengine_hip.h``), called from a host layer that keeps the
reference's operator and engine interfaces.
"""

__version__ = "0.1.0"
