"""Drop-in counterparts of the reference's kernel cases on the MoE dispatch path.

Each module keeps the reference case's entry point -- the bundle's
`kernel_function(*inputs)` (kernel_results/<case>/kernel.py) or the
`reference_*` function of a Contract-B case -- with the same arguments, output
tuple and error behaviour, plus the case's seeded input generator
(`get_inputs` / `make_inputs` / `make_row_id_map`), and runs the HIP kernels of
this package.  Generated inputs are returned on `device` (default "cuda").
"""
from . import (case03_moe_grouped_gemm_fc1_fwd, case04_moe_grouped_gemm_fc2_fwd,  # noqa: F401
               case05_moe_grouped_gemm_fc2_wgrad, case07_moe_grouped_gemm_fc1_dgrad,
               case08_moe_grouped_gemm_fc2_dgrad, case09_moe_grouped_gemm_fc1_wgrad,
               case10_grouped_gemm_single_group_fc1_fwd, case14_grouped_gemm_single_group_fc2_fwd,
               case13_grouped_gemm_single_group_fc1_dgrad, case19_grouped_gemm_single_group_fc2_dgrad,
               case37_ref_musa_asm_bf16_gemm_nn_256x384, case38_ref_musa_asm_bf16_ssgemm_nt_320x256,
               case11_router_bwd_cast_bf16_to_fp32, case25_ref_unary_cast_fp32_to_bf16,
               case31_ref_musa_asm_tf32_ssgemm_tn_128x256, case39_ref_musa_asm_tf32_ssgemm_nn_384x256,
               case06_cp_seq_chunk_index_select, case12_moe_row_id_map_pass2,
               case15_moe_unpermute_mask_fwd, case17_moe_permute_with_mask_map,
               case18_moe_permute_bwd_unpermute_mask, case21_permute_with_mask_map_trans,
               case22_moe_permute_mask_kernel_true, case23_aten_topk,
               case24_moe_unpermute_mask_kernel_false, case30_moe_permute_mask_kernel,
               case32_moe_unpermute_mask_kernel)

ALL = [case03_moe_grouped_gemm_fc1_fwd, case04_moe_grouped_gemm_fc2_fwd, case05_moe_grouped_gemm_fc2_wgrad,
       case07_moe_grouped_gemm_fc1_dgrad, case08_moe_grouped_gemm_fc2_dgrad, case09_moe_grouped_gemm_fc1_wgrad,
       case10_grouped_gemm_single_group_fc1_fwd, case14_grouped_gemm_single_group_fc2_fwd,
       case13_grouped_gemm_single_group_fc1_dgrad, case19_grouped_gemm_single_group_fc2_dgrad,
       case37_ref_musa_asm_bf16_gemm_nn_256x384, case38_ref_musa_asm_bf16_ssgemm_nt_320x256,
       case11_router_bwd_cast_bf16_to_fp32, case25_ref_unary_cast_fp32_to_bf16,
       case31_ref_musa_asm_tf32_ssgemm_tn_128x256, case39_ref_musa_asm_tf32_ssgemm_nn_384x256,
       case06_cp_seq_chunk_index_select,
       case12_moe_row_id_map_pass2, case15_moe_unpermute_mask_fwd, case17_moe_permute_with_mask_map,
       case18_moe_permute_bwd_unpermute_mask, case21_permute_with_mask_map_trans,
       case22_moe_permute_mask_kernel_true, case23_aten_topk, case24_moe_unpermute_mask_kernel_false,
       case30_moe_permute_mask_kernel, case32_moe_unpermute_mask_kernel]
