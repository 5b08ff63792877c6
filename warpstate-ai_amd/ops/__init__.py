"""MI355X (gfx950) implementation of WarpState's BF16 matmul hot path.

Modules keep the reference's names: ``matmul_kernels``, ``matmul_epilogue``,
``matmul_execution`` and ``activation_execution``; ``fused_execution`` holds the fused
entry points the reference composes from separate operators. Kernels live in
``libwarpstate_hip.so`` (``csrc/``), reached through the C ABI of
``include/warpstate_hip.h`` by ``ops._hip``.
"""
