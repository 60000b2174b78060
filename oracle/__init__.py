"""CPU oracle of the vk training hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only
as the checker: nothing in the product (torch-vulkan_amd/) imports, links or calls it, and the product
never falls back to it.

Contents (numpy float64 restatements of the reference's algorithms, plus a C restatement of the
bit-exact parts in oracle/csrc/oracle.c):

  function               follows (reference file:line)                          pinned by (tests/test_oracle.py)
  ---------------------  -----------------------------------------------------  -----------------------------------------------
  round_bf16 / _f16      vkrt/shaders/types.glsl:18-50                          torch .to() on all 2^16 bf16 patterns, halfway
                                                                                cases, subnormals, specials; C restatement
  dequant_int8           vkrt/shaders/dq8.comp.in:39-62,                        golden fixtures, torch closed form, C restatement,
                         torch_vulkan/__init__.py:203-205                       exactness of the fp32 product
  gemm                   vkrt/shaders/mm.comp.in:142-153, csrc/ops_mm.cpp:80-99  torch float64 matmul, identity/zero closed forms
  softmax_fwd / _bwd     vkrt/shaders/softmax.comp.in:27-50                     torch float64 softmax + autograd, row sums,
                                                                                shift invariance, _safe_softmax zero rows
  layer_norm_fwd / _bwd  vkrt/shaders/ln.comp.in:27-81                          torch float64 layer_norm + autograd, moments
  attention_fwd / _bwd   vkrt/shaders/attn.comp.in:210-395,                     torch float64 math SDPA + autograd, Sk=1,
  attention_delta        attn_coop.comp.in:158-301, csrc/ops_attn.cpp:240-248   identical keys, zero dO, lse closed form
  conv2d / _backward     csrc/ops_conv.cpp:60-178, im2col.comp.in              torch float64 conv2d + autograd, delta kernels,
                                                                                adjointness <conv x, g> = <x, conv^T g>
  upsample_nearest / bwd csrc/ops_conv.cpp:185-221, upsample.comp.in            torch F.interpolate + autograd, block sums
  group_norm_fwd / _bwd  csrc/ops_norm.cpp:67-142, gn.comp.in                   torch float64 group_norm + autograd, moments,
                                                                                finite differences
  reduce_sum             csrc/ops_rows.cpp:183-270, reduce.comp.in:27-44       torch float64 sum/mean on strided views, arange
                                                                                closed forms, empty reductions
  ew_map                 vkrt/shaders/ew.comp.in:115-257,                       torch CPU ops at the reference tests' tolerances,
                         tools/gen_shaders.py:53-92, csrc/ops_ew.cpp:146-455    bit equality where CPU rounding is fixed,
                                                                                finite differences of the backward formulas,
                                                                                identities (lerp ends, where, pow by products)
"""

from .ops import (  # noqa: F401
    attention_bwd,
    attention_delta,
    attention_fwd,
    bf16_to_f32,
    conv2d,
    conv2d_backward,
    dequant_int8,
    ew_map,
    EW_EXACT,
    f16_to_f32,
    gemm,
    group_norm_bwd,
    group_norm_fwd,
    layer_norm_bwd,
    layer_norm_fwd,
    reduce_sum,
    rel_l2,
    round_bf16,
    round_f16,
    softmax_bwd,
    softmax_fwd,
    upsample_nearest,
    upsample_nearest_backward,
)
