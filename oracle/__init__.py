"""CPU oracle for the FP4 (E2M1) / INT4 dequant-GEMM path and its MoE variant.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package (`metal-marlin_amd/`)
imports this directory.  It is used by `tests/`, by `__graft_entry__.smoke()`
as the checker, and by `bench.py`'s `cpu_baseline` leg, which times the
reference's own CPU path (torch dequant + fp32 matmul).

Every function restates, in numpy (or torch-CPU for the timed baseline), an
algorithm of RESMP-DEV/metal-marlin and cites the reference file:line it follows.

Pinning status (what checks each function against something other than itself):

* `e2m1_decode`, `dequant_fp4`   -- pinned: FP4_E2M1_BITS table and scale
  known-answers of tests/test_dequant.py, plus an exhaustive closed-form check
  (16 codes x every finite fp16 scale, float64 product, one rounding).
* `dequant_u4`                   -- pinned: magic-bias identity and
  ref_dequant_u4_bulk known answers of tests/test_dequant.py, plus an
  exhaustive q x integral z x sampled s closed-form check.
* `quantize_fp4`                 -- pinned: golden vectors written by importing
  the reference's quantize_fp4.py (tests/golden/make_quantize_fp4_vectors.py),
  plus the nearest-value invariant on random and crafted midpoint inputs.
* `quantize_fp4_calibrated`      -- pinned (tests/test_oracle_quant_cal.py):
  golden vectors of the reference's activation_ranges branch (same script),
  the percentile against an exact-rational order-statistic brute force,
  smooth_factor = 0 and percentile = 100 reducing to the weight-only
  quantizer, act <= 1 scaling the group max by sqrt(act) (exact at act = 1/4
  and 1/16), the float64 scale rounding against a Fraction closed form, and
  the nearest-value invariant of the codes.
* `pack_u4_weights`              -- pinned (tests/test_oracle_pin.py): a
  float64 nearest-integer brute force of q away from ties, crafted groups
  where the float32 scale and its fp16 rounding give different q, exact .5
  ties of w/s + z and of -min/s (half-to-even), and one-signed groups whose
  zero point lies outside [0, 15] and is stored unclipped; also the round-trip
  bound and the reference test-file quantizer on clip-free inputs.
* `flat_quantize`, `flat_dequantize`, `pack_pair` (FP4Metal) -- pinned
  (tests/test_oracle_flat.py): nearest-E2M1 brute force in float64 with ties
  to the lower index, sign from v < 0 (so -0.0 -> code 0), the scale closed
  form and its 1e-8 floor, zero padding of the last group, NaN/inf groups,
  and hand-computed known answers.
* `gemm_fp4_ref`, `gemm_u4_ref`  -- fp32 dequant+matmul; pinned by the
  zero / linearity / all-ones-large-K closed forms of tests/test_gemm.py and a
  brute-force float64 triple loop on tiny shapes.
* MoE (`group_tokens_by_expert`, `gather`, `combine`, `moe_mlp_ref`) --
  pinned by the known-answer cases of tests/test_moe.py and a brute-force
  per-token loop on tiny inputs.
* `router_topk`                  -- pinned (tests/test_oracle_pin.py): a
  float64 per-row softmax with an explicit descending selection, ties to the
  lower expert id, ids compared exactly, on random and crafted tied logits.
"""
