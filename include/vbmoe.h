/*
 * vbmoe.h — C ABI of the MI355X (gfx950) routed-expert MoE engine.
 *
 * One shared library, libvbmoe.so, exports every symbol declared here. Signatures use plain
 * pointers, sizes and ggml type ids only; device pointers are HIP device addresses and every
 * `stream` argument is a hipStream_t passed as void* (NULL = the legacy default stream).
 * All compute entry points are stream-ordered: they enqueue work and return without waiting.
 *
 * Errors: every function returns a vbm_status. A non-zero status leaves a message readable with
 * vbm_last_error() on the calling thread. The mapping mirrors the reference engine's exception
 * contract (tools/engine/expert_dispatch.cpp:25-49, tools/engine/quantized_cuda.cu:220-226):
 * shape, route and residency errors are VBM_ERR_INVALID_ARGUMENT (std::invalid_argument there);
 * device failures and non-finite output are VBM_ERR_RUNTIME (std::runtime_error there).
 *
 * Data formats are ggml's (llama.cpp commit 620d2225, "b11669"):
 *   block_mxfp4 {uint8 e; uint8 qs[16]}   17 B per 32 weights; element i<16 is the low nibble of
 *                                          qs[i], element i>=16 the high nibble of qs[i-16].
 *   block_q8_0  {fp16 d; int8 qs[32]}     34 B per 32 values.
 * Expert banks hold the same bytes re-laid out for 128-bit coalesced loads (see
 * vbm_bank_upload); vbm_bank_export returns the original ggml bytes, bit for bit.
 */
#ifndef VBMOE_H
#define VBMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum vbm_status {
    VBM_OK = 0,
    VBM_ERR_INVALID_ARGUMENT = 1,
    VBM_ERR_RUNTIME = 2,
    VBM_ERR_UNSUPPORTED = 3,
    VBM_ERR_OUT_OF_MEMORY = 4
} vbm_status;

/* ggml type ids (ggml.h enum ggml_type; MXFP4 = 39 per tests/test_cpu_research.py:56). */
enum {
    VBM_TYPE_F32 = 0,
    VBM_TYPE_F16 = 1,
    VBM_TYPE_Q8_0 = 8,
    VBM_TYPE_I32 = 26,
    VBM_TYPE_MXFP4 = 39
};

/* Activation of the expert FFN (tools/engine/f32_experts.hpp:14 F32Activation). */
enum {
    VBM_ACT_SILU = 0,          /* g / (1 + exp(-g)) * u                                  */
    VBM_ACT_SWIGLU_OAI = 1     /* x=min(g,7), y=clamp(u,-7,7): x/(1+exp(-1.702x))*(y+1)   */
};

/* Dot-product accumulation order.
 *   VBM_ORDER_EXACT: the ggml x86 CPU contract — per 32-block integer dots split in eight
 *     4-element lanes, per-lane fp32 FMA chains (even/odd blocks for MXFP4), fixed final tree.
 *     Bit-identical to the CPU vec_dot.
 *   VBM_ORDER_FAST: per-block integer dots are still exact; the fp32 accumulation order is free,
 *     and a fused layer's GLU (gate_up GEMM epilogue) uses a fast exp and divide.
 *     Calls of >= 16 tokens with >= 12 routed rows per expert on average run the MFMA grouped GEMM;
 *     the others run the exact-order GEMV (faster there, and its results satisfy either order). */
enum { VBM_ORDER_EXACT = 0, VBM_ORDER_FAST = 1 };

const char * vbm_last_error(void);
int vbm_abi_version(void);

/* ----------------------------------------------------------------------------------------------
 * Device plumbing (thin wrappers over the HIP runtime so that callers need no HIP headers).
 * -------------------------------------------------------------------------------------------- */
vbm_status vbm_device_count(int * count);
vbm_status vbm_set_device(int device);
vbm_status vbm_device_name(int device, char * name, size_t capacity);
vbm_status vbm_mem_info(size_t * free_bytes, size_t * total_bytes);
vbm_status vbm_malloc(void ** device_ptr, size_t bytes);
vbm_status vbm_free(void * device_ptr);
vbm_status vbm_host_alloc(void ** host_ptr, size_t bytes);  /* pinned (hipHostMalloc)          */
vbm_status vbm_host_free(void * host_ptr);
vbm_status vbm_memcpy_h2d(void * dst, const void * src, size_t bytes, void * stream);
vbm_status vbm_memcpy_d2h(void * dst, const void * src, size_t bytes, void * stream);
vbm_status vbm_memcpy_d2d(void * dst, const void * src, size_t bytes, void * stream);
vbm_status vbm_memset(void * dst, int value, size_t bytes, void * stream);
vbm_status vbm_stream_create(void ** stream);               /* non-blocking, default priority  */
vbm_status vbm_stream_destroy(void * stream);
vbm_status vbm_stream_synchronize(void * stream);
vbm_status vbm_device_synchronize(void);
vbm_status vbm_event_create(void ** event);
vbm_status vbm_event_destroy(void * event);
vbm_status vbm_event_record(void * event, void * stream);
vbm_status vbm_event_synchronize(void * event);
vbm_status vbm_event_query(void * event, int * done);
vbm_status vbm_event_elapsed_ms(void * start, void * stop, float * ms);

/* ----------------------------------------------------------------------------------------------
 * Synthetic inputs. A counter-based generator: every byte is a pure function of
 * (seed, stream id, element index), so host and device produce identical tensors and any subset
 * can be regenerated independently. Float tensors are Box-Muller normals computed in double on
 * the host. Follows the seeded-fixture pattern of tools/trace/make_moe_fixture.py:20-156.
 * -------------------------------------------------------------------------------------------- */
/* MXFP4 expert weights in ggml layout: blocks [first_block, first_block + n_blocks) of tensor
 * `stream`; codes uniform nibbles, exponent byte = 127 + U{exp_lo..exp_hi}. */
vbm_status vbm_synth_mxfp4_host(uint64_t seed, uint64_t stream, uint64_t first_block,
                                uint64_t n_blocks, int exp_lo, int exp_hi, void * dst);
/* Q8_0 weights in ggml layout: int8 codes uniform in [-127,127], fp16 scale = fp16(U(lo,hi)). */
vbm_status vbm_synth_q8_0_host(uint64_t seed, uint64_t stream, uint64_t first_block,
                               uint64_t n_blocks, float scale_lo, float scale_hi, void * dst);
/* fp32 N(mean, std) values [first, first + n) of tensor `stream`. Multithreaded. */
vbm_status vbm_synth_normal_host(uint64_t seed, uint64_t stream, uint64_t first, uint64_t n,
                                 float mean, float std_dev, float * dst);

/* ----------------------------------------------------------------------------------------------
 * Expert banks. A bank holds `n_slots` expert matrices of `rows` x `k` weights of one quantized
 * type (MXFP4 or Q8_0) in device memory, re-laid out in 32-row tiles so that each lane issues
 * 16-byte loads and a wavefront reads whole 1 KiB runs. Byte count per slot equals the ggml byte
 * count (rows * k/32 * 17 or 34); the layout is a permutation, with the exponent byte stored
 * xor 0x80 (= e - 128 as a signed byte). Replaces the device expert bank of
 * Mxfp4NativeCudaDown::Impl (tools/engine/quantized_cuda.cu:367-407) and the llama_moe_cache
 * bank tensors (third_party/patches/llama-b11669-hybrid-experts.patch:2573-2589).
 *
 * Fused gate/up banks (interleave = 1): a 2*I-row expert whose ggml rows [0,I) are gate and
 * [I,2I) up (the fused bank of hybrid-experts.patch:2573-2589) is stored so that each 32-row tile
 * holds gate rows 16t..16t+15 then up rows 16t..16t+15; the fused kernels depend on it.
 * -------------------------------------------------------------------------------------------- */
typedef struct vbm_bank vbm_bank;

vbm_status vbm_bank_create(int type, int64_t rows, int64_t k, int64_t n_slots, int interleave,
                           vbm_bank ** bank);
vbm_status vbm_bank_destroy(vbm_bank * bank);
/* Geometry: bytes of one slot, device base address of the bank. */
vbm_status vbm_bank_info(const vbm_bank * bank, int * type, int64_t * rows, int64_t * k,
                         int64_t * n_slots, size_t * slot_bytes, void ** device_base);
/* Upload one expert (ggml row-major blocks, slot_bytes long) into `slot`. `src` may be host
 * (pageable or pinned) or device memory (`src_on_device`). Host sources are staged through a
 * bounded pinned pool and copied on `stream`; the repack runs on the device. */
vbm_status vbm_bank_upload(vbm_bank * bank, int64_t slot, const void * src, int src_on_device,
                           void * stream);
/* Lossless export of one slot back to ggml bytes (host destination; synchronous on `stream`).
 * Mirrors export_expert (hybrid-experts.patch:2065-2082) and the repack round trip of
 * tests/test_masked_matmul.cpp:59-72. */
vbm_status vbm_bank_export(const vbm_bank * bank, int64_t slot, void * dst_host, size_t capacity,
                           void * stream);
/* Fill slots [first_slot, first_slot + count) on the device with the synthetic generator; the
 * expert in slot s gets ggml blocks starting at (first_expert + s - first_slot) * blocks_per_slot
 * of tensor `stream_id` (identical to vbm_synth_*_host on the same block range). */
vbm_status vbm_bank_generate(vbm_bank * bank, int64_t first_slot, int64_t count,
                             uint64_t seed, uint64_t stream_id, int64_t first_expert,
                             float p0, float p1, void * stream);

/* ----------------------------------------------------------------------------------------------
 * ggml-level operators (drop-in for the ggml ops of the routed-expert branch).
 * -------------------------------------------------------------------------------------------- */

/* quantize_row_q8_0 with the x86 contract restated at
 * third_party/patches/llama-b11669-mxfp4-q8-parity-experimental.patch:41-44,95-96:
 * per 32 values amax, d = fp16_rn(amax/127), q = RNE(x * (127/amax)) (0 when amax == 0).
 * `n_rows` rows of `k` floats (row stride `x_stride` floats) -> n_rows * k/32 blocks. */
vbm_status vbm_quantize_q8_0(const float * x, int64_t n_rows, int64_t k, int64_t x_stride,
                             void * dst_q8, void * stream);

/* GGML_OP_MUL_MAT_ID on a bank (ggml-cpu ggml_compute_forward_mul_mat_id,
 * hybrid-experts.patch:559-640; engine NativeCpuExperts::project, tools/engine/native_cpu.cpp:91-104):
 *   dst[:, r, t] = bank[slot(ids[r,t])] . b[:, r mod b_ne1, t]   (+ bias[:, ids[r,t]] if bias)
 * - ids: int32 [n_ids, n_tokens] with element stride 1 and token stride ids_stride (ints);
 *   -1 zeroes that output row (hybrid-experts.patch:617-621); otherwise 0 <= id < n_as.
 * - expert_to_slot: optional int32 [n_as] device map (NULL = identity); -1 = not resident,
 *   which is an error (VBM_ERR_INVALID_ARGUMENT, checked on the host copy `expert_to_slot_host`
 *   when given).
 * - b: type F32 (quantized on the fly to the bank's vec_dot type, Q8_0) or Q8_0 blocks;
 *   shape [k, b_ne1, n_tokens] contiguous; b_ne1 is 1 (broadcast) or n_ids.
 * - bias: optional fp32 [n_as][rows] (ADD_ID, hybrid-experts.patch:1464-1480).
 * - dst: fp32 [rows, n_ids, n_tokens] contiguous.
 * - order: VBM_ORDER_EXACT or VBM_ORDER_FAST.
 * Uses the device grouping pass (vbm_group_by_expert) so every expert's weights stream once per
 * call, whatever the number of tokens routed to it. Rows of an id outside [-1, n_as), and rows of
 * a routed expert whose expert_to_slot entry is -1 (when no host copy was given to check), come
 * out NaN: the reference asserts on both (hybrid-experts.patch:622; quantized_cuda.cu:224-227).
 * Device scratch: the library keeps one per (device, stream), grown stream-ordered only when a
 * call needs more than any earlier call on that stream, so steady-state calls allocate nothing;
 * a call under graph capture that would grow it fails with VBM_ERR_INVALID_ARGUMENT (run it once
 * on the stream before capturing); vbm_stream_destroy releases it. */
vbm_status vbm_mul_mat_id(const vbm_bank * bank, const int32_t * expert_to_slot,
                          const int32_t * expert_to_slot_host, int64_t n_as,
                          int b_type, const void * b, int64_t b_ne1,
                          const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride,
                          const float * bias, float * dst, int order, void * stream);

/* The same operator over caller-owned device scratch (the ownership of the reference's executor,
 * whose buffers live as long as it does, tools/engine/quantized_cuda.cu:387-400): bytes needed
 * for a call of this shape, then the call itself with `workspace` of at least that size. The
 * workspace holds nothing between calls; calls that share one must not overlap. */
vbm_status vbm_mul_mat_id_workspace(const vbm_bank * bank, int64_t n_as, int64_t b_ne1, int64_t n_ids,
                                    int64_t n_tokens, int order, size_t * bytes);
vbm_status vbm_mul_mat_id_ws(const vbm_bank * bank, const int32_t * expert_to_slot,
                             const int32_t * expert_to_slot_host, int64_t n_as,
                             int b_type, const void * b, int64_t b_ne1,
                             const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride,
                             const float * bias, float * dst, int order, void * workspace,
                             size_t workspace_bytes, void * stream);

/* MUL_MAT_ID without any allocation. No counterpart in the reference: it exists for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same kernels and results as vbm_mul_mat_id, minus the host-copy check of the
 * map (a -1 entry for a routed expert gives NaN rows). Its device scratch is one fixed array of
 * VBM_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends: a call whose shape needs more
 * (vbm_mul_mat_id_workspace reports the need) fails with VBM_ERR_INVALID_ARGUMENT before anything
 * is enqueued. Every call on one GPU shares that array, so calls that overlap on one GPU (on other
 * streams or host threads) race; calls on one stream are ordered and do not. */
#define VBM_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
vbm_status vbm_mul_mat_id_noalloc(const vbm_bank * bank, const int32_t * expert_to_slot, int64_t n_as,
                                  int b_type, const void * b, int64_t b_ne1,
                                  const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride,
                                  const float * bias, float * dst, int order, void * stream);

/* Experimental, outside the parity contract, no counterpart in the reference (its activations are
 * Q8_0): MUL_MAT_ID on an MXFP4 bank with the fp32 activations quantized to MXFP8 (e4m3 codes
 * rounded to nearest even, one e8m0 scale per 32 values: the smallest power of two X with
 * amax / X <= 448, so nothing saturates) and the products on the CDNA4 block-scaled matrix cores
 * (v_mfma_scale_f32_16x16x128_f8f6f4), which apply both block scales in hardware. Results follow the
 * MXFP8 x MXFP4 arithmetic (about 1e-2 relative from the reference's Q8_0 path). b fp32
 * [n_tokens][b_ne1][k] contiguous; ids, expert_to_slot (device map or NULL), -1 ids and dst
 * [n_tokens][n_ids][rows] as in vbm_mul_mat_id (no bias). Device scratch as vbm_mul_mat_id. */
vbm_status vbm_mul_mat_id_mxfp8(const vbm_bank * bank, const int32_t * expert_to_slot, int64_t n_as, const float * b,
                                int64_t b_ne1, const int32_t * ids, int64_t n_ids, int64_t n_tokens,
                                int64_t ids_stride, float * dst, void * stream);
/* The MXFP8 quantizer of vbm_mul_mat_id_mxfp8 alone: n_rows rows of k fp32 (row stride x_stride
 * floats) -> codes [n_rows][k] bytes and e8m0 scales [n_rows][k / 32] bytes. */
vbm_status vbm_quantize_mxfp8(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, void * codes, void * scales,
                              void * stream);

/* GGML_OP_ADD_ID in place: y[:, r, t] += bias[:, ids[r,t]] (rows x n_ids x n_tokens; bias fp32
 * [n_as][rows]). An id of -1 adds nothing; ids outside [-1, n_as) set the row to NaN (the reference
 * asserts on them). */
vbm_status vbm_add_id(float * y, const float * bias, int64_t n_as, const int32_t * ids, int64_t rows,
                      int64_t n_ids, int64_t n_tokens, int64_t ids_stride, void * stream);

/* GGML_OP_GLU swiglu_oai (alpha, limit) and swiglu (SiLU-gated) over n values:
 * out[i] = act(gate[i], up[i]); gate/up/out may use row strides (floats). */
vbm_status vbm_glu(int activation, const float * gate, const float * up, float * out,
                   int64_t n_rows, int64_t width, int64_t gate_stride, int64_t up_stride,
                   int64_t out_stride, float alpha, float limit, void * stream);

/* Router: logits (given, or W_r . x with W_r fp32 [n_expert][k_hidden] and optional bias,
 * computed in the ggml x86 vec_dot_f32 order) -> top-k (value desc, then lower index:
 * tools/trace/topk-tie-probe.cpp:111-113) -> softmax over the k selected
 * (gpt-oss SOFTMAX_WEIGHT gating). If `router_w` is NULL the `logits` input is used;
 * otherwise logits are written to `logits` (may be NULL). ids [n_tokens][k] int32,
 * weights [n_tokens][k] fp32. `normalize` = 0 gives plain softmax-over-selected. */
vbm_status vbm_router_topk_softmax(const float * router_w, const float * router_b,
                                   const float * x, int64_t k_hidden, float * logits,
                                   int64_t n_expert, int64_t n_tokens, int64_t top_k,
                                   int32_t * ids, float * weights, void * stream);

/* Token->expert grouping (the MMID row mapping of hybrid-experts.patch:606-631): a stable
 * counting sort of the (token, rank) pairs by expert.
 *   counts[n_as], offsets[n_as + 1] (exclusive prefix), rows[n_ids*n_tokens] = token*n_ids+rank
 *   listed expert by expert, token-major and rank-minor within an expert. -1 ids are skipped.
 * Invalid ids (outside [-1, n_as)) set *error_flag (device int, optional) to 1; otherwise it is
 * set to 0. Device scratch is the per-stream scratch of vbm_mul_mat_id. */
vbm_status vbm_group_by_expert(const int32_t * ids, int64_t n_ids, int64_t n_tokens,
                               int64_t ids_stride, int64_t n_as, int32_t * counts,
                               int32_t * offsets, int32_t * rows, int32_t * error_flag,
                               void * stream);

/* Weighted top-k combine (hybrid-experts.patch:1905-1924 and :1620-1646; ggml MUL then
 * sequential ADD in rank order): out[:, t] = ((w0*y0 + w1*y1) + w2*y2) + ... with
 * y [rows, n_ids, n_tokens] and weights [n_ids, n_tokens]. */
vbm_status vbm_weighted_combine(const float * y, const float * weights, int64_t rows,
                                int64_t n_ids, int64_t n_tokens, float * out, void * stream);

/* ----------------------------------------------------------------------------------------------
 * Fused routed-expert layer (expert_branch of hybrid-experts.patch:1394-1683 for one layer:
 * gate_up MUL_MAT_ID, bias ADD_ID, GLU, Q8_0 requantization, down MUL_MAT_ID, bias ADD_ID,
 * MUL by the routing weight, rank-ordered sum).
 * -------------------------------------------------------------------------------------------- */
typedef struct vbm_moe_layer_desc {
    const vbm_bank * gate_up;      /* fused 2*I-row bank, interleave = 1                        */
    const vbm_bank * down;         /* H-row bank, k = I                                         */
    const float * gate_up_bias;    /* device, [n_expert][2*I] by expert id, gate | up, or NULL   */
    const float * down_bias;       /* device, [n_expert][H] by expert id, or NULL                */
    const int32_t * expert_to_slot;/* device [n_expert] or NULL (identity)                       */
    const float * router_w;        /* device fp32 [n_expert][H] or NULL (logits given)           */
    const float * router_b;        /* device fp32 [n_expert] or NULL                             */
    int64_t hidden;                /* H                                                          */
    int64_t intermediate;          /* I                                                          */
    int64_t n_expert;
    int64_t top_k;
    int activation;                /* VBM_ACT_*                                                  */
    int order;                     /* VBM_ORDER_*                                                */
} vbm_moe_layer_desc;

/* Workspace bytes needed by vbm_moe_layer_forward for `max_tokens` tokens. */
vbm_status vbm_moe_layer_workspace(const vbm_moe_layer_desc * desc, int64_t max_tokens,
                                   size_t * bytes);

/* x [n_tokens][H] fp32 -> out [n_tokens][H] fp32. `logits` [n_tokens][n_expert] is read when
 * desc->router_w is NULL and written otherwise (may then be NULL). ids/weights (optional,
 * [n_tokens][top_k]) receive the routing. `workspace` is device memory of the size above. */
vbm_status vbm_moe_layer_forward(const vbm_moe_layer_desc * desc, const float * x,
                                 float * logits, int64_t n_tokens, float * out,
                                 int32_t * ids, float * weights, void * workspace,
                                 size_t workspace_bytes, void * stream);

/* Same as vbm_moe_layer_forward, also recording events[0..3] (hipEvent_t as void*) on `stream`
 * immediately before/after the gate_up GEMV and before/after the down GEMV, so callers can time
 * the two dominant kernels over a live run. No reference counterpart (profiling hook, the
 * analogue of the scheduler counters of hybrid-experts.patch:143-172). */
vbm_status vbm_moe_layer_forward_profiled(const vbm_moe_layer_desc * desc, const float * x,
                                          float * logits, int64_t n_tokens, float * out,
                                          int32_t * ids, float * weights, void * workspace,
                                          size_t workspace_bytes, void * const * events,
                                          void * stream);

/* ----------------------------------------------------------------------------------------------
 * Fused single-token decode through a stack of routed-expert layers whose router logits are
 * given (the decode step of llama_decode over build_moe_ffn's routed-expert part,
 * hybrid-experts.patch:1394-1924, for one token). Per layer two kernels run:
 *   A: top-k + softmax routing, the previous layer's weighted rank combine (or the input),
 *      Q8_0 quantization, gate_up GEMV + biases + GLU + Q8_0 requantization;
 *   B: down GEMV + bias;
 * and one final kernel combines the last layer. Each layer's output is bit-identical to
 * vbm_moe_layer_forward with n_tokens = 1. The plan owns its workspace, so a step allocates
 * nothing and can be captured in a HIP graph; steps on one plan must not overlap. All layers
 * share one shape and type; every layer's router_w must be NULL.
 * -------------------------------------------------------------------------------------------- */
typedef struct vbm_decode_plan vbm_decode_plan;

vbm_status vbm_decode_plan_create(const vbm_moe_layer_desc * layers, int64_t n_layers,
                                  vbm_decode_plan ** plan);
vbm_status vbm_decode_plan_destroy(vbm_decode_plan * plan);
/* x [hidden] (16-byte aligned) -> out [hidden]; logits [n_layers][n_expert]; ids / weights
 * optional [n_layers][top_k] outputs. events: optional [n_layers][4] hipEvent_t (as void*)
 * recorded before/after kernel A and before/after kernel B of every layer (NULL: none). */
vbm_status vbm_decode_step(vbm_decode_plan * plan, const float * x, const float * logits,
                           float * out, int32_t * ids, float * weights, void * const * events,
                           void * stream);
/* One kernel of one layer of the step (which = 0: kernel A, 1: kernel B) on the plan's current
 * state, for timing and profiling a kernel in isolation; both are idempotent, so repeated
 * launches stream the same bytes. */
vbm_status vbm_decode_kernel(vbm_decode_plan * plan, int64_t layer, int which, const float * x,
                             const float * logits, void * stream);
/* Linked step (no reference counterpart: a launch schedule of the same arithmetic), opt-in for
 * MXFP4 layers with hidden = intermediate = 2880 and at most 128 experts: a step runs
 * n_layers + 1 launches, launch j holding the down tiles of layer j - 1 and the gate_up tiles of
 * layer j, which wait on device-side per-tile flags for their input instead of a kernel boundary.
 * Outputs are bit-identical to the two-kernel step (the default, which is faster on MI355X: the
 * flag round trips queue behind the weight streams). events then holds [n_layers + 1][2] records
 * around the launches. set_linked(plan, 1) fails with VBM_ERR_INVALID_ARGUMENT for other shapes. */
vbm_status vbm_decode_plan_set_linked(vbm_decode_plan * plan, int linked);
vbm_status vbm_decode_plan_get_linked(const vbm_decode_plan * plan, int * linked);
/* Synchronizes the device, then reports and clears the device waits of linked steps that timed
 * out since the last check (*timeouts, optional): VBM_ERR_RUNTIME if any did, since that step's
 * outputs are unspecified. A wait times out after about 0.17 s. */
vbm_status vbm_decode_plan_check(vbm_decode_plan * plan, int64_t * timeouts);

/* ----------------------------------------------------------------------------------------------
 * Causal expert admission over one shared pool of n_slots expert slots serving n_layers routed
 * layers (host-side control state; no device calls). Restates llama_moe_cache::admit
 * (third_party/patches/llama-b11669-hybrid-experts.patch:3087-3242), write_dispatch (:3059-3084)
 * and the admission helpers (:3543-3574). Slots [0, n_used) are the reserved per-rank zero slots
 * of misses; anchors follow them (vbm_admission_set_anchors). Keys are layer * n_expert + expert.
 * -------------------------------------------------------------------------------------------- */
#define VBM_ADMIT_CLASSIC 0  /* recent-frequency margin, lowest-recent victim (the default)   */
#define VBM_ADMIT_LRU 1      /* free slot or least recently seen; the reference uses margin 1   */
#define VBM_ADMIT_RANKED 2   /* classic with seed-priority / recency tie-breaks                 */
#define VBM_ADMIT_PROBATION 3 /* classic; margin 4 + (3 - reuse) after an unreused lifetime   */
#define VBM_ADMIT_ANCHORED 4 /* classic above a floor protecting up to 1/4 of the pool for seeds */
#define VBM_ADMIT_LFU 5      /* capped demand counts, periodic halving, LRU victim              */

typedef struct vbm_admission vbm_admission;

vbm_status vbm_admission_create(int64_t n_layers, int64_t n_expert, int64_t n_used, int64_t n_slots,
                                int64_t recent_window, int32_t margin, int policy,
                                vbm_admission ** out);
vbm_status vbm_admission_destroy(vbm_admission * a);
/* Frozen-plan seed (llama-b11669-hybrid-experts.patch:2659-2680): the next free slot from n_used
 * upward; earlier seeds get the higher seed priority. Only before the first dispatch. */
vbm_status vbm_admission_seed(vbm_admission * a, int64_t layer, int64_t expert, int32_t * slot);
/* Reserve `anchors` protected slots after the zero slots (admission floor = n_used + anchors). */
vbm_status vbm_admission_set_anchors(vbm_admission * a, int32_t anchors);
/* One single-token dispatch of `layer`: selected[n_used] expert ids in rank order. hits[n_used]
 * (optional) receives residency before admission; the admissions made are returned in order as
 * (admitted_slots[i], admitted_experts[i], evicted_keys[i] or -1), i < *n_admitted <= n_used. */
vbm_status vbm_admission_admit(vbm_admission * a, int64_t layer, const int32_t * selected,
                               int32_t * hits, int32_t * admitted_slots, int32_t * admitted_experts,
                               int32_t * evicted_keys, int64_t * n_admitted);
/* Dispatch packing for n_tokens tokens: ids / weights [n_tokens][n_used] -> out
 * [n_tokens][4][n_used] = (-1 or cpu expert id, slot or rank, 0 or weight, 0 or 1 miss mask);
 * cold_rank >= 0 sends token 0's rank to the transient scratch slot n_slots. */
vbm_status vbm_admission_write_dispatch(const vbm_admission * a, int64_t layer, const int32_t * ids,
                                        const float * weights, int64_t n_tokens, int32_t cold_rank,
                                        float * out);
vbm_status vbm_admission_slot_map(const vbm_admission * a, int64_t layer, int32_t * map);
/* stats[4] = dispatch calls, hits before admission, admissions, evictions. */
vbm_status vbm_admission_stats(const vbm_admission * a, uint64_t * stats);

/* LFU thresholds (llama-b11669-hybrid-experts.patch:2199-2200, :2398-2413): demands before an
 * expert may replace a cached one (default 6) / take a free slot (default 1), each in 1..15. */
vbm_status vbm_admission_set_lfu(vbm_admission * a, int32_t admit_after, int32_t fill_after);

/* LFU demand counts [n_layers * n_expert] (may be NULL) and the number of halvings so far
 * (:2191-2195); for inspection and tests. No reference counterpart beyond those fields. */
vbm_status vbm_admission_lfu_state(const vbm_admission * a, uint16_t * counts, uint64_t * halvings);
/* llama_moe_colder_admission / probation_margin / anchor_slots / cold_gpu_budget /
 * gpu_slot_limit; -1 where the reference asserts. */
int vbm_moe_colder_admission(int candidate_frequency, int candidate_seed_priority,
                             uint64_t candidate_last_seen, int current_frequency,
                             int current_seed_priority, uint64_t current_last_seen);
int vbm_moe_probation_margin(int observed_lifetime, uint64_t future_hits);
int vbm_moe_anchor_slots(int capacity, int reserved, int seeds);
int vbm_moe_cold_gpu_budget(int cold_experts);
int32_t vbm_moe_gpu_slot_limit(int32_t resident_slots, int cold_gpu);

/* Offline residency replay of a decode routing trace under the expert-cache cost models of the
 * reference's analyzer (tools/benchmark/vrambridge-routing.py:191-512): events in trace order,
 * layer indices in ascending layer-id order, experts of event i at [event_offsets[i],
 * event_offsets[i + 1]); event_split 0 = training request (warms the cache), 1 = held-out
 * request (totalled). Host-side. */
#define VBM_RESIDENCY_MEASURED_STATIC 0
#define VBM_RESIDENCY_TRAIN_STATIC 1
#define VBM_RESIDENCY_LRU 2
#define VBM_RESIDENCY_LFU 3
#define VBM_RESIDENCY_BELADY_HITS 4
#define VBM_RESIDENCY_COST_AWARE 5

typedef struct {
    int64_t experts;
    uint64_t bytes_per_expert, static_host_bytes_per_expert;
} vbm_residency_layer;

typedef struct {
    int policy;                              /* VBM_RESIDENCY_*                                  */
    uint64_t capacity_bytes;
    int admit_after;                         /* references before admission (>= 1)             */
    int64_t payback_tokens;                  /* cost-aware window in generated tokens (>= 1)   */
    int cold_cache;                          /* clear the cache before the first held-out event */
    double ram_gbps, pcie_gbps, gpu_expert_us, layer_sync_us;
    int staging_ram_passes;                  /* 0 or 2                                          */
    uint64_t static_device_expert_bytes;     /* the trace metadata's (measured_static)          */
} vbm_residency_params;

typedef struct {
    int supported;                           /* 0: belady_hits over unequal expert sizes        */
    uint64_t expert_calls, full_hits, bytes, cold_bytes, upload_bytes, evictions;
    double serial_s, optimistic_s, shared_ram_bytes;   /* latency-model sums over held-out layers */
    uint64_t warmup_upload_bytes, initial_bytes, rejected, warmup_rejected;
} vbm_residency_totals;

vbm_status vbm_residency_replay(const vbm_residency_layer * layers, int64_t n_layers, const int32_t * event_layer,
                                const int32_t * event_split, const int64_t * event_offsets, const int32_t * experts,
                                int64_t n_events, const vbm_residency_params * params, vbm_residency_totals * totals);
/* The latency model alone (Costs.latency, vrambridge-routing.py:212-223) for one layer's cold
 * bytes, GPU experts and uploads, with params' costs: serial, optimistic-overlap seconds and the
 * shared RAM bytes. */
vbm_status vbm_residency_latency(const vbm_residency_params * params, double cpu_bytes, double gpu_experts,
                                 double upload_bytes, double * serial_s, double * optimistic_s, double * shared_ram_bytes);

/* ----------------------------------------------------------------------------------------------
 * GGUF expert tensors (tools/engine/gguf_experts.cpp:27-140): blk.L.ffn_{gate,up,down}_exps.
 * {weight,bias} (or the fused blk.L.ffn_gate_up_exps.weight) of a GGUF file and its
 * "-0000k-of-0000N.gguf" shards, read one expert slice at a time. Headers are parsed at open;
 * tensor data is read on demand with pread. Weights must be MXFP4 or Q8_0, biases F32.
 * -------------------------------------------------------------------------------------------- */
typedef struct vbm_gguf vbm_gguf;

typedef struct {
    int64_t hidden, intermediate, n_expert;
    int gate_up_type, down_type;             /* ggml type ids                                    */
    int fused_gate_up;                       /* ffn_gate_up_exps instead of separate gate / up   */
    int has_bias;
    uint64_t gate_up_bytes, down_bytes;      /* ggml bytes of one expert (gate rows then up rows) */
} vbm_gguf_expert_info;

/* path: a single .gguf or the first shard "<stem>-00001-of-NNNNN.gguf" (then all NNNNN are read). */
vbm_status vbm_gguf_open(const char * path, vbm_gguf ** gguf);
vbm_status vbm_gguf_close(vbm_gguf * gguf);
vbm_status vbm_gguf_shards(const vbm_gguf * gguf, int64_t * shards, int64_t * tensors);
/* Metadata of integer (or bool) / string keys. found == NULL makes a missing key an error. */
vbm_status vbm_gguf_get_u64(const vbm_gguf * gguf, const char * key, uint64_t * value, int * found);
vbm_status vbm_gguf_get_string(const vbm_gguf * gguf, const char * key, char * dst, size_t capacity, int * found);
/* ne[4] ggml dimensions; nbytes 0 for types of unknown block size. */
vbm_status vbm_gguf_tensor_info(const vbm_gguf * gguf, const char * name, int * type, int64_t * ne,
                                uint64_t * nbytes, int * found);
vbm_status vbm_gguf_expert_layer_info(const vbm_gguf * gguf, int64_t layer, vbm_gguf_expert_info * info);
/* Host copies of one expert: ggml bytes of gate|up (gate_up_bytes) and down (down_bytes), fp32
 * biases gate|up [2I] and down [H] (zeros when the file has none). Any output may be NULL. */
vbm_status vbm_gguf_read_expert(const vbm_gguf * gguf, int64_t layer, int64_t expert, void * gate_up,
                                void * down, float * gate_up_bias, float * down_bias);
/* experts[n] of `layer` into bank slots[n] (NULL: slot = expert id) of a fused interleaved gate_up
 * bank and a down bank, plus every expert's biases into device arrays indexed by expert id
 * (either may be NULL). Synchronous on `stream` for the biases. */
vbm_status vbm_gguf_load_layer(const vbm_gguf * gguf, int64_t layer, const int32_t * experts,
                               const int32_t * slots, int64_t n, vbm_bank * gate_up, vbm_bank * down,
                               float * gate_up_bias, float * down_bias, void * stream);
vbm_status vbm_gguf_load_biases(const vbm_gguf * gguf, int64_t layer, float * gate_up_bias,
                                float * down_bias, void * stream);

/* ----------------------------------------------------------------------------------------------
 * Decode routing traces in the reference's JSONL schema (benchmarks/schema/
 * vrambridge-routing-trace.schema.json), written like its collector tools/trace/routing_trace.cpp:
 * metadata (:701-728), request_start (:501-503), one route per routed layer and decoded token
 * (:206-216), request_end (:566-569), trace_end (:744). Records are compact JSON lines with keys in
 * ascending order; the file is written as "<path>.part" (created exclusively) and hard-linked to
 * `path` by vbm_trace_close (:632-634, :745-749). Host-side; no device calls.
 * -------------------------------------------------------------------------------------------- */
typedef struct {
    int64_t id;                              /* model layer number                               */
    int64_t experts, active;                 /* experts in the layer, experts routed per token   */
    uint64_t bytes_per_expert;               /* all expert tensors of the layer, per expert      */
    uint64_t static_host_bytes_per_expert;   /* of which statically held in host memory          */
    const char * tensor_types;               /* comma-separated ggml type names, or NULL         */
} vbm_trace_layer;

typedef struct vbm_trace vbm_trace;

/* model, token_equivalence_check and collector_source_sha256 (64 lower-case hex digits) may be
 * NULL (omitted). Refuses an existing path or partial. */
vbm_status vbm_trace_open(const char * path, const char * architecture, const char * backend_commit,
                          const char * model, int64_t context_tokens, const vbm_trace_layer * layers,
                          int64_t n_layers, const char * token_equivalence_check,
                          const char * collector_source_sha256, vbm_trace ** trace);
/* Also write the prefill summary of the reference collector's prefill mode (routing_trace.cpp:
 * 750-769: "observed_prefill_expert_rows", pretty-printed, published like the trace) to
 * summary_path at vbm_trace_close. Before the first request; needs collector_source_sha256. */
vbm_status vbm_trace_enable_prefill(vbm_trace * trace, const char * summary_path, int64_t batch_size,
                                    int64_t microbatch_size, int64_t cpu_threads, int64_t batch_threads);
vbm_status vbm_trace_prefill_enabled(const vbm_trace * trace, int * enabled);
/* One prompt batch of `layer_id` in the open request, before its decode routes: ids [rows][active]
 * (0..32768 rows; 0 records an output-pruned batch), each row's experts in range and distinct;
 * recorded as the batch's rows-per-expert histogram (routing_trace.cpp:180-225). Before the first
 * decode route (or request end) every routed layer must have seen 1..prompt_tokens rows
 * (routing_trace.cpp:510-519); the request's coverage is written at request end. */
vbm_status vbm_trace_prefill_route(vbm_trace * trace, int64_t layer_id, const int32_t * ids, int64_t rows);
/* split "train" or "test"; prompt_tokens + max_tokens <= context_tokens; ids unique. */
vbm_status vbm_trace_request_start(vbm_trace * trace, const char * id, const char * split,
                                   const char * category, int64_t prompt_tokens, int64_t max_tokens);
/* One layer's routed experts (rank order) for the current token; layers in ascending id order. */
vbm_status vbm_trace_route(vbm_trace * trace, int64_t layer_id, const int32_t * experts, int64_t n_active);
/* All layers of one token: ids [n_layers][stride] (stride 0 = each layer's active count), e.g. the
 * ids output of vbm_decode_step or vbm_tier_step copied to the host. */
vbm_status vbm_trace_token(vbm_trace * trace, const int32_t * ids, int64_t stride);
/* stop_reason "limit" (exactly max_tokens decoded) or "eos" (fewer); token_sequence_equivalent
 * non-zero records the observer-equivalence claim, zero omits it. */
vbm_status vbm_trace_request_end(vbm_trace * trace, const char * stop_reason, int token_sequence_equivalent);
/* Writes trace_end and publishes the file. Consumes the handle, also on failure. */
vbm_status vbm_trace_close(vbm_trace * trace);
/* Discards the partial file and the handle. */
vbm_status vbm_trace_abort(vbm_trace * trace);
/* Layer `index` in ascending id order; any output may be NULL. */
vbm_status vbm_trace_layer_info(const vbm_trace * trace, int64_t index, int64_t * id, int64_t * experts,
                                int64_t * active);
/* Routed layers, requests started, complete tokens of the open request (-1: none open), next
 * layer index within the current token. */
vbm_status vbm_trace_position(const vbm_trace * trace, int64_t * n_layers, int64_t * requests,
                              int64_t * token, int64_t * layer_index);

/* ----------------------------------------------------------------------------------------------
 * Single-GPU host-RAM expert tier for single-token decode (the cold-expert path of the reference's
 * llama_moe_cache: admission, staged uploads and publish-after-event,
 * llama-b11669-hybrid-experts.patch:2727-3298). Every expert of every layer is kept in pinned
 * host memory in the device bank layout; n_slots device slots shared by all layers hold the
 * resident set under causal admission; the first top_k of them (the admission's reserved zero
 * slots) stage the current layer's remaining misses. Misses are computed on the GPU after their
 * copy (no CPU expert path). A step synchronizes once per layer (the routing must reach the host
 * before the admission), so it cannot be captured in a graph.
 * -------------------------------------------------------------------------------------------- */
typedef struct {
    int type;                            /* VBM_TYPE_MXFP4 or VBM_TYPE_Q8_0 */
    int64_t hidden, intermediate, n_layers, n_expert, top_k;
    int activation;
    int64_t n_slots;                     /* device pool in expert groups (> top_k) */
    int64_t recent_window;               /* admission history, in dispatches per layer (8..256) */
    int32_t margin;
    int policy;                          /* VBM_ADMIT_* */
    const float * const * gate_up_bias;  /* host array of n_layers device pointers, or NULL */
    const float * const * down_bias;     /* host array of n_layers device pointers, or NULL */
} vbm_tier_desc;

typedef struct {
    uint64_t dispatches, hits, admissions, evictions, staged, uploaded_bytes;
    double copy_ms;                      /* copy-stream busy time (events around each layer's copies) */
    uint64_t prefill_tokens;             /* tokens through vbm_tier_prefill                       */
    uint64_t prefill_resident;           /* routed experts computed from resident slots (per call) */
    uint64_t prefill_streamed;           /* routed experts streamed through the reserved slots    */
    uint64_t host_reads;                 /* deferred mode: routed experts the decode kernels read  */
                                         /* from the pinned host copy (not visible in the map)    */
    uint64_t device_copy_bytes;          /* deferred mode: bytes copied on the device to admit    */
                                         /* experts (staging area -> slot; no host upload)         */
} vbm_tier_stats;

typedef struct vbm_tier vbm_tier;

vbm_status vbm_tier_create(const vbm_tier_desc * desc, vbm_tier ** tier);
vbm_status vbm_tier_destroy(vbm_tier * tier);
/* Pinned host bytes the tier holds (all experts of all layers). */
vbm_status vbm_tier_host_bytes(const vbm_tier * tier, size_t * bytes);
/* Store one expert from ggml bytes (gate|up rows then down rows of block_mxfp4 / block_q8_0). */
vbm_status vbm_tier_set_expert(vbm_tier * tier, int64_t layer, int64_t expert, const void * gate_up_ggml,
                               const void * down_ggml, void * stream);
/* Store every expert from the seeded generator of vbm_bank_generate: layer l's gate|up experts
 * use stream id layer_stride * l + gate_up_stream, its down experts layer_stride * l + down_stream.
 * Both stores must precede seeding and stepping. */
vbm_status vbm_tier_generate(vbm_tier * tier, uint64_t seed, uint64_t layer_stride, uint64_t gate_up_stream,
                             uint64_t down_stream, float p0, float p1, void * stream);
/* Store every expert of GGUF layers layer_ids[n_layers] (tier layer l <- GGUF layer layer_ids[l]);
 * shapes and types must match the tier. Biases stay the caller's (vbm_gguf_load_biases). */
vbm_status vbm_tier_load_gguf(vbm_tier * tier, const vbm_gguf * gguf, const int64_t * layer_ids, void * stream);
/* Frozen-plan seed: admit (layer, expert) into the next slot and copy it there. */
vbm_status vbm_tier_seed(vbm_tier * tier, int64_t layer, int64_t expert);
/* x [hidden] (16-byte aligned) -> out [hidden]; logits [n_layers][n_expert]; ids optional
 * [n_layers][top_k]. Bit-identical to vbm_decode_step on resident banks holding the same experts. */
vbm_status vbm_tier_step(vbm_tier * tier, const float * x, const float * logits, float * out, int32_t * ids,
                         void * stream);
/* Multi-token prefill of one layer (16..65536 tokens; the MFMA grouped GEMM, VBM_ORDER_FAST):
 * x [T][hidden] (16-byte aligned) -> out [T][hidden]; logits [T][n_expert]; ids / weights optional
 * [T][top_k]. Residency is frozen for the batch (no admission; the reference freezes it for
 * multi-position dispatch, llama-b11669-hybrid-experts.patch:3252-3257): the routed experts
 * resident in the pool are computed from their slots in one pass, and the others stream through
 * the reserved slots in chunks of top_k / 2, each chunk's copies on the side stream overlapping
 * the previous chunk's GEMMs. This is the device-side counterpart of the reference's
 * resident-down prefill split (llama-b11669-resident-down-prefill-experimental.patch:192-283),
 * which runs cold experts on the CPU instead. Outputs are bit-identical to
 * vbm_moe_layer_forward (VBM_ORDER_FAST) over banks holding every expert. */
vbm_status vbm_tier_prefill(vbm_tier * tier, int64_t layer, const float * x, const float * logits,
                            int64_t n_tokens, float * out, int32_t * ids, float * weights, void * stream);
vbm_status vbm_tier_get_stats(const vbm_tier * tier, vbm_tier_stats * stats);
/* Empties the pool (every slot free) and restarts admission with the given policy, window and
 * margin and zeroed stats, keeping the host copies: a new run over the same experts without
 * re-storing them. Seeds, if any, follow with vbm_tier_seed. */
vbm_status vbm_tier_reset(vbm_tier * tier, int policy, int64_t recent_window, int64_t margin);
/* Deferred mode (enable = 1; 0 returns to the synchronous per-layer mode), the device-side
 * counterpart of the reference's hosted flush (llama-b11669-hybrid-experts.patch:2953-3005) and
 * event-protected ID hand-off (:3421-3453): a step's layers run back to back with no host wait,
 * reading each layer's expert->slot map from the device; a routed expert that is not visible
 * there is read once from the pinned host copy by the decode kernels, which keep a copy of it in
 * a device staging area ([n_layers][top_k] expert copies, allocated when the mode is enabled);
 * the step's routed ids come back behind an event, and the next step (or vbm_tier_flush) runs
 * admission on them, copies each admitted expert from the staging area into its slot (device to
 * device: an admitted expert crosses PCIe once) and publishes it in the same flush. Admission
 * sees the same routes in the same order as the synchronous mode, so the counters (staged
 * included: the misses that mode would stage) and outputs are the same; `host_reads` counts the
 * routed experts the kernels read from host memory (exactly the misses). Stats lag one step until
 * vbm_tier_flush. No routing trace is recorded in this mode. */
vbm_status vbm_tier_set_deferred(vbm_tier * tier, int enable);
/* Deferred mode: waits for the step in flight, runs its admission and publishes every upload. */
vbm_status vbm_tier_flush(vbm_tier * tier);
/* Deferred mode, vbm_tier_step split in two: the host part (the flush above) and the device part,
 * which makes no host call and may be captured in a HIP graph once and replayed after each
 * vbm_tier_step_begin (its map upload and id hand-off read and write the tier's pinned buffers at
 * replay time). Every begin is followed by exactly one enqueue or replay before the next begin or
 * flush: the next begin admits that step's routed ids. */
vbm_status vbm_tier_step_begin(vbm_tier * tier);
vbm_status vbm_tier_step_enqueue(vbm_tier * tier, const float * x, const float * logits, float * out, int32_t * ids,
                                 void * stream);

/* Attach a routing trace (or NULL to detach): every vbm_tier_step then records each layer's
 * routed experts, as they reach the host for admission, as one route record (tier layer l is the
 * trace's l-th layer in ascending id order; counts and top_k must match). When the trace writes
 * a prefill summary, every vbm_tier_prefill also records its routed ids as prompt batches of
 * <= 32768 rows (vbm_trace_prefill_route). The trace stays owned by the caller and must outlive
 * the attachment. */
vbm_status vbm_tier_set_trace(vbm_tier * tier, vbm_trace * trace);

/* ----------------------------------------------------------------------------------------------
 * Stream-ordered host calls: the HIP side of the reference's GGML_OP_CUSTOM host-call node
 * (struct ggml_host_call, third_party/patches/llama-b11669-hybrid-experts.patch:82-101, and the
 * CUDA backend's handling of it, :800-1054). vbm_host_call has ggml_host_call's layout (with
 * VBM_HOST_MAX_SRC equal to GGML_MAX_SRC), so a ggml HIP backend passes the node's userdata
 * straight through. fn runs on a host thread and must not call device APIs; src_host[i] and
 * dst_host are pinned host buffers (vbm_host_alloc) of the input and output sizes.
 * -------------------------------------------------------------------------------------------- */
#define VBM_HOST_CALL_MAGIC 0x56424843414c4c31ULL /* "VBHCALL1" */
#define VBM_HOST_JOIN_MAGIC 0x5642484a4f494e31ULL /* "VBHJOIN1" */
#define VBM_HOST_MAX_SRC 10
#define VBM_HOST_CALL_FUNC 0      /* hipLaunchHostFunc on the side stream                        */
#define VBM_HOST_CALL_MAILBOX 1   /* device-posted request to a persistent host worker (bounded) */

typedef struct vbm_host_call {
    uint64_t magic;
    void (*fn)(void * ctx);
    void * ctx;
    void * src_host[VBM_HOST_MAX_SRC];
    void * dst_host;
    void * backend_state;           /* owned by the library once the call has been enqueued      */
    struct vbm_host_call * call;    /* join nodes: the call they wait for                        */
    int32_t miss_src;               /* ggml's field; the miss ids are passed to the enqueue here */
} vbm_host_call;

/* Creates the call's events, the device's side stream and (mailbox) its worker: do it before
 * capturing a graph that enqueues the call. */
vbm_status vbm_host_call_prepare(vbm_host_call * call, int mode);
/* On a side stream forked from `stream`: device srcs[i] (src_bytes[i]) -> call->src_host[i],
 * fn(ctx), call->dst_host -> device dst (dst_bytes). miss (mailbox mode, optional): device int32
 * [n_miss]; when none of them is 0 the call is posted for bookkeeping only, not waited for, and dst
 * is zero-filled (fn still runs before vbm_host_mailbox_drain returns). The call runs on the side
 * stream: work that needs its output, or a synchronize meant to cover it, must follow a
 * vbm_host_join or vbm_host_call_wait on `stream`. */
vbm_status vbm_host_call_enqueue(vbm_host_call * call, const void * const * srcs, const size_t * src_bytes,
                                 int n_src, void * dst, size_t dst_bytes, const int32_t * miss, int64_t n_miss,
                                 int mode, void * stream);
/* Join node: dst = a + b (fp32, n) on `stream` once the call has completed. */
vbm_status vbm_host_join(vbm_host_call * call, const float * a, const float * b, float * dst, int64_t n,
                         void * stream);
/* Makes `stream` wait for the call's completion without a join. */
vbm_status vbm_host_call_wait(vbm_host_call * call, void * stream);
/* Waits for the call's last enqueue, and for the worker to have run fn for its last mailbox post
 * (also one that was not waited for; bounded, VBM_ERR_RUNTIME on expiry), then frees what the
 * library attached to it. Re-enqueuing a descriptor is safe too: in either mode the new input
 * copies wait on the device (bounded) until the worker has handled the call's previous post. */
vbm_status vbm_host_call_release(vbm_host_call * call);
/* Returns once the device's worker has handled every posted request (call after the stream is idle). */
vbm_status vbm_host_mailbox_drain(int device, double timeout_s);
/* Requests posted and handled, and waited posts whose bounded wait expired (output zero-filled). */
vbm_status vbm_host_mailbox_stats(int device, uint64_t * posted, uint64_t * done, uint32_t * timeouts);
/* Polls (~1 us each) a waited post makes before it expires; default 2^21. */
vbm_status vbm_host_mailbox_set_spin_limit(uint32_t polls);

/* ----------------------------------------------------------------------------------------------
 * ggml backend boundary: supports_op and compute_forward over ggml-layout graph nodes.
 * The reference builds the routed-expert branch as ggml nodes
 * (third_party/patches/llama-b11669-hybrid-experts.patch:1394-1683: MUL_MAT_ID, ADD_ID, gate/up
 * views, GLU, MUL_MAT_ID, ADD_ID, MUL by the routing weights; :1905-1916: ADD of the resident and
 * host halves, sequential ADDs of strided rank views, CONT; :966-1054: CUSTOM host calls;
 * :1860-1916: the frozen-hybrid dispatch, whose packed slot remap (vbm_admission_write_dispatch)
 * reaches MUL_MAT_ID through strided views and I32 casts) and
 * hands each node to a backend through compute_forward (:1079-1083) and supports_op (:1101-1102; the
 * pattern of fp32-experts-experimental.patch:74-82). vbm_node carries ggml_tensor's fields: a
 * backend adapter copies type, ne, nb, data, op_params and src from its tensor, sets `op` to the
 * VBM_NODE_* value of the tensor's ggml op, and sets `extra`:
 *   - on a MUL_MAT_ID's src[0] (the expert tensor): a vbm_expert_tensor binding its bank;
 *   - on a CUSTOM node: its host-call or join descriptor (a vbm_host_call), the node's userdata.
 * Strides are byte strides (ggml nb); data pointers are device pointers.
 * -------------------------------------------------------------------------------------------- */
#define VBM_NODE_MAX_SRC 10
#define VBM_NODE_NONE 0          /* leaf: no compute                                              */
#define VBM_NODE_VIEW 1          /* VIEW / RESHAPE / PERMUTE / TRANSPOSE: no compute              */
#define VBM_NODE_ADD 2           /* dst = src0 + src1 (src1 repeated over src0), F32, any strides */
#define VBM_NODE_MUL 3           /* dst = src0 * src1 (src1 repeated over src0), F32, any strides */
#define VBM_NODE_CONT 4          /* dst (contiguous) = src0 in its element order, F32             */
#define VBM_NODE_MUL_MAT_ID 5    /* src0 expert tensor, src1 b, src2 ids (see vbm_mul_mat_id)     */
#define VBM_NODE_ADD_ID 6        /* src0 y, src1 bias [rows, n_as], src2 ids (see vbm_add_id)     */
#define VBM_NODE_GLU 7           /* src0 gate (src1 up, or the second half of src0's rows)        */
#define VBM_NODE_CUSTOM 8        /* host call or host join (extra = vbm_host_call)                */
#define VBM_NODE_CPY 9           /* ggml_cast: contiguous dst = src0 converted, F32 <-> I32       */
/* ggml_glu_op values (GLU op_params[0]); op_params[1] = swapped; SWIGLU_OAI: op_params[2] alpha
 * and op_params[3] limit, as float bits (ggml_swiglu_oai). */
#define VBM_GLU_OP_SWIGLU 2
#define VBM_GLU_OP_SWIGLU_OAI 3

typedef struct vbm_node {
    int32_t op;                              /* VBM_NODE_*                                       */
    int32_t type;                            /* VBM_TYPE_* (ggml type id)                         */
    int64_t ne[4];                           /* ggml ne, ne[0] fastest                            */
    size_t nb[4];                            /* ggml nb, bytes                                    */
    void * data;                             /* device pointer                                    */
    void * extra;                            /* see above                                         */
    int32_t op_params[16];                   /* ggml op_params (GGML_MAX_OP_PARAMS / 4)           */
    const struct vbm_node * src[VBM_NODE_MAX_SRC];
} vbm_node;

/* The bank that holds an expert tensor, with its optional expert->slot maps (as in vbm_mul_mat_id). */
typedef struct vbm_expert_tensor {
    const vbm_bank * bank;
    const int32_t * expert_to_slot;          /* device int32 [ne[2]] or NULL (identity)            */
    const int32_t * expert_to_slot_host;     /* host copy for checking, or NULL                    */
} vbm_expert_tensor;

typedef struct vbm_compute_params {
    int32_t order;                           /* VBM_ORDER_* for MUL_MAT_ID                        */
    int32_t host_call_mode;                  /* VBM_HOST_CALL_FUNC or VBM_HOST_CALL_MAILBOX       */
} vbm_compute_params;

/* supports_op: 1 when this library can run the node with its types, shapes and strides
 * (MUL_MAT_ID: MXFP4/Q8_0 experts [k % 64, rows % 32, n_as <= 1024]; F32 b with evenly spaced
 * rows, any row stride, or contiguous Q8_0 b; I32 ids with contiguous rows and any token stride;
 * contiguous F32 dst. GLU: gate/up rows evenly spaced, so the split views of a fused gate_up
 * qualify. ADD / MUL / CONT / ADD_ID: F32 with any 4-byte strides). */
int vbm_node_supported(const vbm_node * node);
/* compute_forward: runs one node on `stream` (params NULL: exact order, hipLaunchHostFunc host
 * calls). A node vbm_node_supported refuses fails with VBM_ERR_UNSUPPORTED and the reason. */
vbm_status vbm_compute_forward(const vbm_node * node, const vbm_compute_params * params, void * stream);
/* The nodes of a graph in order (views and leaves are skipped); the first failure names its node. */
vbm_status vbm_graph_compute(const vbm_node * const * nodes, int64_t n_nodes, const vbm_compute_params * params,
                             void * stream);

/* ----------------------------------------------------------------------------------------------
 * HIP graph capture of stream-ordered work (per-token layer chains replay without host launch
 * overhead). Only entry points that do not allocate (the layer forward with a caller workspace,
 * the router, combine, quantize and device copies) may be captured.
 * -------------------------------------------------------------------------------------------- */
vbm_status vbm_graph_begin_capture(void * stream);
vbm_status vbm_graph_end_capture(void * stream, void ** graph_exec);
vbm_status vbm_graph_launch(void * graph_exec, void * stream);
vbm_status vbm_graph_destroy(void * graph_exec);

/* Plain streaming copy kernel (16 B per lane); a known-size HBM reference for counter scaling. */
vbm_status vbm_copy_kernel(void * dst, const void * src, size_t bytes, void * stream);

#ifdef __cplusplus
}
#endif

#endif /* VBMOE_H */
