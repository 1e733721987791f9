"""DeepSeek-V2-Lite decode kernels for MI355X (gfx950), hand-written in HIP.

Same module and function names as the reference's ``triton_kernels`` package
(rmsnorm, attention_prepost, mlp_elementwise, moe_router, moe_batch,
moe_small_gemv, attention_decode_batch, attention_decode_small); there is no
Triton here -- every function calls the C ABI of libdsv2lite_hip.so through
``triton_kernels._hip`` and raises if that library is not built.
"""
