"""mmfp4 -- MI355X (gfx950) FP4-E2M1 / INT4 dequant-GEMM and MoE grouped-expert
path with the Python surface of RESMP-DEV/metal-marlin's quantized linear,
kernels and moe_dispatch modules.  Kernels live in libmmfp4.so (HIP, C ABI)."""

from .kernels import (FP4_PER_UINT, decode_gemv_fp4, dequant_fp4, dequant_fp4_decode_gemv,
                      dequant_int4, dequantize_mmfp4, fused_gate_up_gemm, marlin_gemm_fp4,
                      marlin_gemm_fp4_tuned, marlin_gemm_fused_fp4, marlin_gemm_fused_u4,
                      marlin_gemm_int4, mmfp4_fused_gate_up, mmfp4_fused_gate_up_marlin,
                      mmfp4_fused_qkv,
                      mmfp4_gemm, mmfp4_gemm_rowpacked, rowpacked_gemm_supported,
                      select_decode_kernel)
from .gpu_grouping import (GPUExpertGrouping, GPUGroupingResult, group_tokens_by_expert_auto,
                           group_tokens_by_expert_fast, group_tokens_by_expert_gpu_optimized)
from .fp4_metal import FP4Metal, dequantize_fp4_metal, quantize_fp4_metal
from .layers import MMFP4Linear
from .ops import GemmFp4, dispatch_gemm_fp4
from .loader import QuantizedModel, convert_safetensors_to_fp4, load_and_quantize_safetensors
from .moe_dispatch import (FusedMoEDispatcher, MoEDispatcher, _fused_expert_mlp,
                           dispatch_experts_batched, moe_add_shared_expert_fp4,
                           moe_fused_dispatch_shared_fp4, moe_shared_expert_fp4,
                           moe_shared_expert_fused_fp4, MoEDispatchInfo, compute_expert_load,
                           compute_load_balancing_loss, gather_for_experts,
                           group_tokens_by_expert, group_tokens_by_expert_full,
                           fused_router_topk, mmfp4_softmax_topk, moe_expert_gemm_fp4,
                           moe_fused_router_sorted, moe_mlp_fp4, moe_router_topk,
                           router_softmax_topk,
                           scatter_expert_outputs)
from .quantize_fp4 import (E2M1_VALUES, compute_quantization_error, pack_u4_weights,
                           quantize_fp4, unpack_fp4, unpack_u4_weights)
from .quantized_linear import (KernelLibrary, MarlinLinear, QuantizedLinear, QuantizedTensor,
                               dequant_fp4_bulk, dequant_int4_bulk, get_default_library,
                               quantized_linear)

from ._lib import release_workspaces

__version__ = "0.1.0"
