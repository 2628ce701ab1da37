"""omnistack_rs — MI355X (gfx950) build of OmniStack-RS's KV-cache codec and
compressed-KV attention.

Same module layout and call signatures as the reference package
(deepsheth3/Omnistack-RS ``omnistack_rs``): ``kernels.hadamard``,
``kernels.quantize``, ``kernels.fused_attention``, ``quantization``,
``attention``, ``config``.  The hot path (rotation, encode, decode,
attention, LoRA) runs hand-written HIP kernels through the C ABI of
``_native/libomnistack_amd.so``; it needs HIP device tensors.
"""

__version__ = "0.1.0"
