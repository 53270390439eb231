"""MI355X-native (gfx950) GGUF quantized-linear hot path behind Tensor's runtime contract.

``tensor_amd.Device(provider="hip")`` opens a HIP device session whose built-in
executables are the hand-written GGUF kernels of ``libtensor_hip.so``:

    import tensor_amd as tx
    with tx.Device(provider="hip") as device:
        linear = device.load("gguf_linear", encoding="q4_k", out_dtype="float16")
        out = linear(x_buffer, w_buffer)          # allocates out, launches async
"""

from tensor_amd.providers import PROVIDERS, Device

__all__ = ["Device", "PROVIDERS"]
__version__ = "0.1.0"
