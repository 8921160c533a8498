/*
 * Compiled against the reference's own headers (sdk/include/pai/op.h,
 * ir/ir.h) and linked with the registry built from its sources: the layout
 * claims of include/pai_hip.h are checked by the compiler, the descriptors
 * register and resolve, and the selection a GGUF-aware kernel choice makes
 * (the executor change shown in INTEGRATION.md) finds them.
 */
#include <stddef.h>
#include <stdio.h>
#include <string.h>

#include <pai/op.h>

#include "cpu/reference/ref_ops.h"
#include "ir/ir.h"
#include "models/quantize.h"
#include "pai_hip.h"

#define SAME_FIELD(A, B, f)                                                                    \
  _Static_assert(offsetof(A, f) == offsetof(B, f) && sizeof(((A *)0)->f) == sizeof(((B *)0)->f), \
                 #f)

_Static_assert(sizeof(pai_hip_op_descriptor_t) == sizeof(pai_op_descriptor_t), "descriptor size");
SAME_FIELD(pai_hip_op_descriptor_t, pai_op_descriptor_t, name);
SAME_FIELD(pai_hip_op_descriptor_t, pai_op_descriptor_t, version);
SAME_FIELD(pai_hip_op_descriptor_t, pai_op_descriptor_t, num_inputs);
SAME_FIELD(pai_hip_op_descriptor_t, pai_op_descriptor_t, num_outputs);
SAME_FIELD(pai_hip_op_descriptor_t, pai_op_descriptor_t, in_dtype);
SAME_FIELD(pai_hip_op_descriptor_t, pai_op_descriptor_t, out_dtype);
SAME_FIELD(pai_hip_op_descriptor_t, pai_op_descriptor_t, caps);
SAME_FIELD(pai_hip_op_descriptor_t, pai_op_descriptor_t, ref_fn);
SAME_FIELD(pai_hip_op_descriptor_t, pai_op_descriptor_t, kernel_id);
SAME_FIELD(pai_hip_op_descriptor_t, pai_op_descriptor_t, reserved);
_Static_assert((PAI_OP_CAP_GPU_HIP & (PAI_OP_CAP_CPU_REF | PAI_OP_CAP_GPU_SERIAL |
                                      PAI_OP_CAP_HOST_REF)) == 0,
               "the HIP bit is free");

_Static_assert(sizeof(pai_hip_ir_quant_t) == sizeof(pai_ir_quant_t), "quant size");
SAME_FIELD(pai_hip_ir_quant_t, pai_ir_quant_t, present);
SAME_FIELD(pai_hip_ir_quant_t, pai_ir_quant_t, bit_width);
SAME_FIELD(pai_hip_ir_quant_t, pai_ir_quant_t, scale_repr);
SAME_FIELD(pai_hip_ir_quant_t, pai_ir_quant_t, zero_point_repr);
SAME_FIELD(pai_hip_ir_quant_t, pai_ir_quant_t, is_signed);
SAME_FIELD(pai_hip_ir_quant_t, pai_ir_quant_t, block_structure);
SAME_FIELD(pai_hip_ir_quant_t, pai_ir_quant_t, group_size);
/* the proposed block structure is the next free value of the enum */
_Static_assert(PAI_IR_QUANT_BLOCK_GGUF == (unsigned)PAI_IR_QUANT_BLOCK_COUNT, "next value");
_Static_assert(PAI_IR_QUANT_REPR_F16 == 1, "f16 repr value");

/* v0 schemes and GEMMs: the same record and the same prototypes */
_Static_assert(sizeof(pai_hip_quant_scheme_t) == sizeof(pai_quant_scheme_t), "scheme size");
SAME_FIELD(pai_hip_quant_scheme_t, pai_quant_scheme_t, bit_width);
SAME_FIELD(pai_hip_quant_scheme_t, pai_quant_scheme_t, is_signed);
SAME_FIELD(pai_hip_quant_scheme_t, pai_quant_scheme_t, group_size);
#define SAME_TYPE(a, b) _Static_assert(__builtin_types_compatible_p(__typeof__(&a), __typeof__(&b)), #a)
SAME_TYPE(pai_hip_gemm_w8_f32, pai_ref_gemm_w8_f32);
SAME_TYPE(pai_hip_gemm_w4_f32, pai_ref_gemm_w4_f32);
SAME_TYPE(pai_gemm_w8_ref_f32, pai_ref_gemm_w8_f32);
SAME_TYPE(pai_gemm_w4_ref_f32, pai_ref_gemm_w4_f32);

/* What a GGUF-aware pai_kernel_select resolves a GEMM to: the weight's tag
 * picks the qgemm descriptor, an untagged weight keeps matmul_f32. */
static const char *gemm_op_name(const pai_hip_ir_quant_t *weight_tag) {
  const uint32_t t = pai_hip_quant_type(weight_tag);
  return t != 0u ? pai_hip_op_name(t) : "matmul_f32";
}

int main(void) {
  pai_op_registry_t reg;
  if (pai_op_registry_builtin(&reg) != PAI_OK) return 1;
  uint32_t n = 0;
  const pai_hip_op_descriptor_t *d = pai_hip_op_descriptors(&n);
  for (uint32_t i = 0; i < n; ++i)
    if (pai_op_registry_register(&reg, (const pai_op_descriptor_t *)&d[i]) != PAI_OK) return 2;
  const uint32_t types[4] = {PAI_QTYPE_Q4_0, PAI_QTYPE_Q8_0, PAI_QTYPE_Q4_K, PAI_QTYPE_Q6_K};
  for (int i = 0; i < 4; ++i) {
    pai_hip_ir_quant_t tag;
    if (pai_hip_quant_tag(types[i], &tag) != PAI_OK) return 3;
    /* the tag passes the IR's own validation once the enum has the value */
    if (tag.block_structure != PAI_IR_QUANT_BLOCK_GGUF || tag.bit_width == 0u) return 4;
    const pai_op_descriptor_t *op = pai_op_registry_lookup(&reg, gemm_op_name(&tag));
    if (op == NULL || op != (const pai_op_descriptor_t *)&d[i]) return 5;
    if (!pai_op_supports(op, PAI_OP_CAP_CPU_REF) || !pai_op_supports(op, PAI_OP_CAP_GPU_HIP))
      return 6;
    if (op->ref_fn != (pai_op_ref_fn)pai_qgemm_ref_f32) return 7;
  }
  /* the v0 GEMMs: three inputs as the builtin gemm_w8_f32 / gemm_w4_f32,
   * whose entries stay in place */
  const char *v0[2] = {"qgemm_w8_f32", "qgemm_w4_f32"};
  const pai_op_ref_fn v0_ref[2] = {(pai_op_ref_fn)pai_gemm_w8_ref_f32,
                                   (pai_op_ref_fn)pai_gemm_w4_ref_f32};
  for (int i = 0; i < 2; ++i) {
    const pai_op_descriptor_t *op = pai_op_registry_lookup(&reg, v0[i]);
    if (op == NULL || op->num_inputs != 3u || op->ref_fn != v0_ref[i]) return 10;
    if (!pai_op_supports(op, PAI_OP_CAP_CPU_REF) || !pai_op_supports(op, PAI_OP_CAP_GPU_HIP))
      return 11;
  }
  if (pai_op_registry_lookup(&reg, "gemm_w8_f32") == NULL ||
      pai_op_registry_lookup(&reg, "gemm_w4_f32") == NULL)
    return 12;
  pai_hip_ir_quant_t plain;
  memset(&plain, 0, sizeof plain);
  if (strcmp(gemm_op_name(&plain), "matmul_f32") != 0) return 8;
  if (pai_op_registry_lookup(&reg, gemm_op_name(&plain)) == NULL) return 9;
  printf("boundary ok: %u descriptors\n", n);
  return 0;
}
