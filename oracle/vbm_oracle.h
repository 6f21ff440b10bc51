/*
 * vbm_oracle.h — CPU oracle for the routed-expert MoE path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library,
 * and only as the checker / the timed CPU baseline; the product (libvbmoe.so) never links it.
 *
 * It restates, in plain C, the CPU arithmetic the reference's hot path relies on (ggml x86 at
 * llama.cpp commit 620d2225, as restated inside the reference repository). Each function cites
 * the reference lines it follows. Every function exists in a scalar form; the *_fast entry
 * points (AVX2/FMA/F16C or AVX-512 VNNI, multithreaded) must return identical bits and are
 * checked against the scalar form by the tests.
 *
 * Parts marked "parity unpinned" below have no golden vector, known answer or buildable reference
 * in the reference repository (they live in upstream ggml, which it does not vendor); what the
 * mathematics fixes is still tested for them:
 *   orc_vec_dot_q8_0_q8_0  chain structure across blocks unpinned (one FMA chain per lane, as the
 *                          upstream AVX2 dot); integer block dot pinned by brute force, lane
 *                          arithmetic + tree bit-equal to the reference's compiled MXFP4 dot on
 *                          equivalent inputs, result within its float64 error bound
 *   orc_vec_dot_f32        summation order unpinned (router logits come from upstream
 *                          ggml_mul_mat); within its float64 error bound, hand-derived order
 *                          probes; router ids equal the float64 top-k wherever the gaps exceed
 *                          the worst-case error of any fp32 order
 *   orc_softmax_selected   ggml soft_max expf bits unpinned (closed forms tested)
 * orc_glu is pinned bit for bit against the reference executor's activation
 * (tools/engine/f32_experts.cpp:68-73) compiled into oracle/_ref with the same libm.
 */
#ifndef VBM_ORACLE_H
#define VBM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_TYPE_F32 0
#define ORC_TYPE_Q8_0 8
#define ORC_TYPE_MXFP4 39
#define ORC_ACT_SILU 0
#define ORC_ACT_SWIGLU_OAI 1

int orc_abi_version(void);
float orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16(float f);
float orc_e8m0_half(uint8_t e);

/* quantize_row_q8_0, x86 contract. */
void orc_quantize_row_q8_0(const float * x, void * y, int64_t k);

/* ggml_vec_dot_mxfp4_q8_0 (n % 64 == 0). */
float orc_vec_dot_mxfp4_q8_0(int n, const void * vx, const void * vy);
/* Exact integer dot of one MXFP4 block with one Q8_0 block per the 8-lane VPSIGNB contract;
 * lanes[8] receives the per-lane integers. */
int32_t orc_mxfp4_block_lanes(const void * vx, const void * vy, int32_t lanes[8]);
/* ggml_vec_dot_q8_0_q8_0 (AVX2 contract). */
float orc_vec_dot_q8_0_q8_0(int n, const void * vx, const void * vy);
int32_t orc_q8_block_lanes(const void * vx, const void * vy, int32_t lanes[8]);
/* ggml_vec_dot_f32 (x86 AVX2 order). */
float orc_vec_dot_f32(int n, const float * x, const float * y);

/* GGML_OP_MUL_MAT_ID (as in vbm_mul_mat_id, ggml layout for `as`). threads <= 0: scalar. */
int orc_mul_mat_id(int type, const void * as, int64_t k, int64_t rows, int64_t n_as,
                   int b_type, const void * b, int64_t b_ne1,
                   const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride,
                   const float * bias, float * dst, int threads);

/* Stable counting sort of (token, rank) pairs by expert. Returns 0, or -1 on an invalid id. */
int orc_group_by_expert(const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride,
                        int64_t n_as, int32_t * counts, int32_t * offsets, int32_t * rows);

/* Canonical top-k (value desc, then lower index). */
void orc_topk(const float * logits, int64_t n, int64_t k, int32_t * ids);
/* ggml soft_max over the k selected logits (double sum, float scale). */
void orc_softmax_selected(const float * values, int64_t k, float * out);
/* Router: logits (given, or W.x + b) -> top-k -> softmax-over-selected for n_tokens. */
void orc_router(const float * router_w, const float * router_b, const float * x, int64_t hidden,
                float * logits, int64_t n_expert, int64_t n_tokens, int64_t top_k,
                int32_t * ids, float * weights);

/* GLU: out = act(gate, up). */
void orc_glu(int activation, const float * gate, const float * up, float * out, int64_t n,
             float alpha, float limit);

/* Weighted rank-ordered combine: out[:,t] = ((w0*y0 + w1*y1) + ...). */
void orc_weighted_combine(const float * y, const float * weights, int64_t rows, int64_t n_ids,
                          int64_t n_tokens, float * out);

/* One routed-expert layer (the reference expert_branch graph), weights in ggml layout:
 * gate_up [n_expert][2I rows][H] (rows [0,I) gate, [I,2I) up), down [n_expert][H][I],
 * biases fp32 or NULL. x [T][H] -> out [T][H]. act_out (optional) [T][k][I] receives the GLU
 * output before requantization, y_out (optional) [T][k][H] the biased down outputs. */
typedef struct orc_layer {
    int type;                      /* ORC_TYPE_MXFP4 or ORC_TYPE_Q8_0 */
    const void * gate_up;
    const void * down;
    const float * gate_up_bias;    /* [n_expert][2I] or NULL */
    const float * down_bias;       /* [n_expert][H] or NULL  */
    const float * router_w;        /* [n_expert][H] or NULL  */
    const float * router_b;        /* [n_expert] or NULL     */
    int64_t hidden, intermediate, n_expert, top_k;
    int activation;
} orc_layer;

int orc_moe_layer(const orc_layer * layer, const float * x, float * logits, int64_t n_tokens,
                  float * out, int32_t * ids, float * weights, float * act_out, float * y_out,
                  int threads);

/* Secondary CPU contract (repacked 8x8, tools/trace/exact_packed_cpu.h:52-88): block_mxfp4x8
 * packing of 8-row groups (inverse of the export at HP:751-762) and the one-row GEMV over it.
 * out[nc] for nc rows (nc % 8 == 0); returns -1 on shapes the reference rejects (:80). */
void orc_pack_mxfp4x8(const void * raw_rows, int64_t rows, int64_t blocks, void * packed);
void orc_unpack_mxfp4x8(const void * packed, int64_t rows, int64_t blocks, void * raw_rows);
int orc_gemv_mxfp4x8_q8_0(int n, float * out, const void * packed, const void * act, int nc);

/* Fast (bit-identical) single-row dots used by orc_mul_mat_id when threads > 0. */
int orc_fast_isa(void);  /* 0 scalar, 2 AVX2, 3 AVX-512 VNNI */

#ifdef __cplusplus
}
#endif

#endif
