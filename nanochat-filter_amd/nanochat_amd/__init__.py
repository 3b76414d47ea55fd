"""MI355X (gfx950) implementation of nanochat-filter's LTV combined-QKV path.

Module names under this package mirror the reference's ``nanochat`` package
(``nanochat/ltv_combined_qkv_computer_module.py``,
``nanochat/ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter.py``,
``nanochat/ops/ltv_cuda_ops.py`` ...), so the filter can be swapped into the
reference's ``gpt.py`` / ``gpt_factory.py`` by changing the import root.

The compute runs in ``libnanochat_filter_amd.so`` (hand-written HIP for gfx950,
C ABI in ``include/nanochat_filter_amd.h``), loaded by ``nanochat_amd._native``.
"""

__all__ = ["ops"]
