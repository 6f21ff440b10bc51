// The ggml backend boundary: which graph nodes a HIP backend may hand to this library (the
// supports_op half of a backend; the compute half calls vbm_mul_mat_id / vbm_add_id / vbm_glu /
// vbm_host_call_enqueue / vbm_host_join). Shapes are ggml ne[4] in ggml order (ne[0] fastest).
// Mirrors what the reference's HIP-less CUDA path accepts for these nodes on the routed-expert
// branch (third_party/patches/llama-b11669-hybrid-experts.patch:559-640 MUL_MAT_ID semantics,
// :1464-1480 ADD_ID, :1586-1593 GLU, :966-988 host-call / join nodes), restricted to the types and
// shapes the kernels here implement.
#include "vbm_internal.hpp"

using namespace vbm;

extern "C" {

int vbm_op_supported(int op, int type0, int type1, const int64_t * ne0, const int64_t * ne1) {
    if (!ne0) return 0;
    switch (op) {
        case VBM_OP_MUL_MAT_ID:
            // as: [k, rows, n_as, 1] MXFP4/Q8_0 bank; b: [k, 1 or n_ids, n_tokens, 1] F32/Q8_0
            return (type0 == VBM_TYPE_MXFP4 || type0 == VBM_TYPE_Q8_0) &&
                   (type1 == VBM_TYPE_F32 || type1 == VBM_TYPE_Q8_0) && ne1 != nullptr &&
                   ne0[0] > 0 && ne0[0] % 64 == 0 && ne0[1] > 0 && ne0[1] % 32 == 0 && ne0[2] >= 1 &&
                   ne0[2] <= 1024 && ne0[3] == 1 && ne1[0] == ne0[0] && ne1[1] >= 1 && ne1[2] >= 1 && ne1[3] == 1;
        case VBM_OP_ADD_ID:
            // y: [rows, n_ids, n_tokens, 1] F32; bias: [rows, n_as, 1, 1] F32
            return type0 == VBM_TYPE_F32 && type1 == VBM_TYPE_F32 && ne1 != nullptr && ne0[0] > 0 && ne0[1] >= 1 &&
                   ne0[2] >= 1 && ne0[3] == 1 && ne1[0] == ne0[0] && ne1[1] >= 1 && ne1[2] == 1 && ne1[3] == 1;
        case VBM_OP_GLU_SWIGLU:
        case VBM_OP_GLU_SWIGLU_OAI:
            // split gate / up of [width, rows, ...] F32 each (ne1: the up operand's shape)
            return type0 == VBM_TYPE_F32 && type1 == VBM_TYPE_F32 && ne1 != nullptr && ne0[0] > 0 &&
                   ne1[0] == ne0[0] && ne1[1] == ne0[1] && ne1[2] == ne0[2] && ne1[3] == ne0[3];
        case VBM_OP_HOST_JOIN:
            // dst = a + b, F32, same shape
            return type0 == VBM_TYPE_F32 && type1 == VBM_TYPE_F32 && ne1 != nullptr &&
                   ne0[0] == ne1[0] && ne0[1] == ne1[1] && ne0[2] == ne1[2] && ne0[3] == ne1[3];
        default:
            return 0;
    }
}

}  // extern "C"
