"""MI355X-native AWQ W4A16 dequant-GEMM (gfx950 HIP kernels behind a C ABI) with the
reference's Python call surface for that path."""
from . import _lib, ops  # noqa: F401
from .awq import AWQConfig  # noqa: F401
from .awq_fused_gemm import (  # noqa: F401
    awq_decode_gemv_enabled,
    awq_fused_gate_up_enabled,
    awq_fused_gate_up_group32_enabled,
    awq_fused_gemm,
    awq_fused_gemm_safe,
    packed_int4_symmetric_fused_gate_up_group32_m1,
    packed_int4_symmetric_fused_gate_up_m1,
    packed_int4_symmetric_fused_gate_up_m1_safe,
    packed_int4_symmetric_fused_qkv_m1,
    packed_int4_symmetric_fused_qkv_m1_safe,
    packed_int4_symmetric_fused_qkv_m2,
    packed_int4_symmetric_fused_qkv_m2_safe,
    packed_int4_symmetric_fused_gemm,
    packed_int4_symmetric_fused_gemm_safe,
    packed_int4_symmetric_group32_rows_exact_msmall_safe,
)
from .awq_triton import (  # noqa: F401
    awq_dequantize_triton,
    awq_fused_capability_check,
    awq_gemm_triton,
    packed_int4_fused_capability_check,
)
from .fused_pair import try_fused_awq_gate_up_activation, try_fused_awq_pair_matmul  # noqa: F401
from .moe import (  # noqa: F401
    AWQExperts,
    awq_moe,
    fused_moe,
    gemma4_moe_int4_prefill_grouped,
    gemma4_moe_int4_prefill_grouped_fused,
    moe_route,
)
from .rmsnorm_awq_fused import rmsnorm_awq_fused_linear  # noqa: F401
from .tensor import AWQWeight, PackedInt4Weight  # noqa: F401

__version__ = "0.1.0"
