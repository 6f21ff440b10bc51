// The ggml backend boundary for the routed-expert branch: supports_op and compute_forward over
// ggml-layout graph nodes (vbm_node: type, ne[4], nb[4] byte strides, data, op, op_params, src[]).
//
// The reference builds the branch at third_party/patches/llama-b11669-hybrid-experts.patch:1394-1683
// (MUL_MAT_ID -> ADD_ID -> gate/up views -> GLU -> MUL_MAT_ID -> ADD_ID -> MUL by the routing
// weights) and joins ranks at :1905-1916 (ADD of the resident and host halves, then sequential ADDs
// of strided rank views, then CONT); a backend claims each node through supports_op and runs it in
// compute_forward (:1079-1083, :1101-1102; the pattern of fp32-experts-experimental.patch:74-82). The node
// rules below follow the ggml CPU semantics of each op (:559-640 for MUL_MAT_ID), restricted to
// what the kernels here implement; strides are checked, so a view the kernels cannot read is
// refused by the predicate instead of being read wrongly.
#include "vbm_internal.hpp"

#include <cstring>
#include <string>

using namespace vbm;

namespace {

// ---------------------------------------------------------------------------------------------
// Elementwise kernels over ggml byte strides (one thread per element of the output shape)
// ---------------------------------------------------------------------------------------------

struct Dims {
    int64_t ne[4];
};
struct Strides {
    int64_t nb[4];   // bytes
};

enum { EW_ADD = 0, EW_MUL = 1, EW_COPY = 2 };

__device__ __forceinline__ void unflatten(int64_t idx, const Dims & d, int64_t (&i)[4]) {
    i[0] = idx % d.ne[0];
    idx /= d.ne[0];
    i[1] = idx % d.ne[1];
    idx /= d.ne[1];
    i[2] = idx % d.ne[2];
    i[3] = idx / d.ne[2];
}

__device__ __forceinline__ int64_t offset(const int64_t (&i)[4], const Strides & s) {
    return i[0] * s.nb[0] + i[1] * s.nb[1] + i[2] * s.nb[2] + i[3] * s.nb[3];
}

// dst = a (op) b, b repeated over a's shape (ggml_can_repeat broadcast); EW_COPY: dst = a.
template <int OP>
__global__ void elementwise_kernel(char * dst, Strides sd, const char * a, Strides sa,
                                   const char * b, Strides sb, Dims shape, Dims b_shape, int64_t n) {
    for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < n;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t i[4];
        unflatten(idx, shape, i);
        const float x = *reinterpret_cast<const float *>(a + offset(i, sa));
        float v = x;
        if constexpr (OP != EW_COPY) {
            const int64_t j[4] = {i[0] % b_shape.ne[0], i[1] % b_shape.ne[1], i[2] % b_shape.ne[2], i[3] % b_shape.ne[3]};
            const float y = *reinterpret_cast<const float *>(b + offset(j, sb));
            v = OP == EW_ADD ? x + y : x * y;
        }
        *reinterpret_cast<float *>(dst + offset(i, sd)) = v;
    }
}

// GGML_OP_ADD_ID: dst[i0, i1, i2] = a[i0, i1, i2] + bias[i0, ids[i1, i2]]. An id of -1 adds
// nothing (the masked ranks of the resident branch); an id outside [-1, n_as) gives NaN (the
// reference asserts on it).
__global__ void add_id_kernel(char * dst, Strides sd, const char * a, Strides sa,
                              const char * __restrict__ bias, int64_t bias_nb1, int64_t n_as,
                              const char * __restrict__ ids, int64_t ids_nb0, int64_t ids_nb1, Dims shape, int64_t n) {
    for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < n;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t i[4];
        unflatten(idx, shape, i);
        const int32_t id = *reinterpret_cast<const int32_t *>(ids + i[1] * ids_nb0 + i[2] * ids_nb1);
        const float x = *reinterpret_cast<const float *>(a + offset(i, sa));
        float v = x;
        if (id >= 0 && id < n_as)
            v = x + *reinterpret_cast<const float *>(bias + id * bias_nb1 + i[0] * static_cast<int64_t>(sizeof(float)));
        else if (id != -1)
            v = __builtin_nanf("");
        *reinterpret_cast<float *>(dst + offset(i, sd)) = v;
    }
}

// GGML_OP_CPY (ggml_cast): element idx of src's row-major order goes to element idx of dst's,
// converted between F32 and I32. F32 -> I32 truncates toward zero, the C conversion ggml's CPU
// cast applies; where C leaves it undefined, out-of-range values saturate and NaN gives 0 here.
// I32 -> F32 rounds to nearest.
__global__ void convert_kernel(char * dst, Strides sd, Dims dshape, int dst_i32, const char * a, Strides sa,
                               Dims ashape, int src_i32, int64_t n) {
    for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < n;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t i[4], j[4];
        unflatten(idx, ashape, i);
        unflatten(idx, dshape, j);
        const char * s = a + offset(i, sa);
        char * d = dst + offset(j, sd);
        if (src_i32) {
            const int32_t v = *reinterpret_cast<const int32_t *>(s);
            if (dst_i32) *reinterpret_cast<int32_t *>(d) = v;
            else *reinterpret_cast<float *>(d) = static_cast<float>(v);
        } else {
            const float v = *reinterpret_cast<const float *>(s);
            if (dst_i32)
                *reinterpret_cast<int32_t *>(d) = v != v ? 0
                                                 : v >= 2147483648.0f ? INT32_MAX
                                                 : v <= -2147483648.0f ? INT32_MIN : static_cast<int32_t>(v);
            else *reinterpret_cast<float *>(d) = v;
        }
    }
}

unsigned grid_for(int64_t n) {
    const int64_t blocks = (n + 255) / 256;
    return static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
}

Dims dims_of(const int64_t * ne) { return Dims{{ne[0], ne[1], ne[2], ne[3]}}; }
Strides strides_of(const size_t * nb) {
    return Strides{{static_cast<int64_t>(nb[0]), static_cast<int64_t>(nb[1]), static_cast<int64_t>(nb[2]),
                    static_cast<int64_t>(nb[3])}};
}

// ---------------------------------------------------------------------------------------------
// ggml tensor geometry
// ---------------------------------------------------------------------------------------------

struct TypeInfo {
    int64_t blck = 0;
    int64_t size = 0;
};

TypeInfo type_info(int type) {
    switch (type) {
        case VBM_TYPE_F32: return {1, 4};
        case VBM_TYPE_F16: return {1, 2};
        case VBM_TYPE_I32: return {1, 4};
        case VBM_TYPE_Q8_0: return {32, 34};
        case VBM_TYPE_MXFP4: return {32, 17};
        default: return {};
    }
}

int64_t nelements(const vbm_node & t) { return t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]; }

bool shape_valid(const vbm_node & t) {
    const TypeInfo ti = type_info(t.type);
    if (ti.blck == 0) return false;
    for (int d = 0; d < 4; ++d)
        if (t.ne[d] < 1 || t.ne[d] > (int64_t(1) << 40)) return false;
    return t.ne[0] % ti.blck == 0 && nelements(t) <= (int64_t(1) << 40);
}

// ggml_nbytes
size_t nbytes(const vbm_node & t) {
    const TypeInfo ti = type_info(t.type);
    size_t bytes = ti.blck == 1 ? static_cast<size_t>(ti.size) : static_cast<size_t>(t.ne[0] / ti.blck) * t.nb[0];
    for (int d = ti.blck == 1 ? 0 : 1; d < 4; ++d) bytes += static_cast<size_t>(t.ne[d] - 1) * t.nb[d];
    return bytes;
}

// ggml_is_contiguous: dims of extent 1 place no constraint on their stride.
bool contiguous(const vbm_node & t) {
    const TypeInfo ti = type_info(t.type);
    size_t next = static_cast<size_t>(ti.size);
    if (t.ne[0] != ti.blck && t.nb[0] != next) return false;
    next *= static_cast<size_t>(t.ne[0] / ti.blck);
    for (int d = 1; d < 4; ++d) {
        if (t.ne[d] == 1) continue;
        if (t.nb[d] != next) return false;
        next *= static_cast<size_t>(t.ne[d]);
    }
    return true;
}

// An F32 tensor whose elements are contiguous within a row and whose rows (dims 1..3 flattened,
// dim 1 fastest) are evenly spaced: row r starts at data + r * row_stride. The stride is returned
// in floats.
bool uniform_rows(const vbm_node & t, int64_t * row_stride) {
    if (t.type != VBM_TYPE_F32 || (t.ne[0] > 1 && t.nb[0] != sizeof(float))) return false;
    int64_t stride = -1;
    size_t next = 0;
    for (int d = 1; d < 4; ++d) {
        if (t.ne[d] == 1) continue;
        if (stride < 0) {
            if (t.nb[d] % sizeof(float) != 0) return false;
            stride = static_cast<int64_t>(t.nb[d] / sizeof(float));
        } else if (t.nb[d] != next) {
            return false;
        }
        next = t.nb[d] * static_cast<size_t>(t.ne[d]);
    }
    if (stride < 0) stride = t.ne[0];
    if (stride < t.ne[0]) return false;   // rows must not overlap
    *row_stride = stride;
    return true;
}

bool aligned_strides(const vbm_node & t) {
    for (int d = 0; d < 4; ++d)
        if (t.nb[d] % sizeof(float) != 0) return false;
    return (reinterpret_cast<uintptr_t>(t.data) & (sizeof(float) - 1)) == 0;
}

bool same_shape(const vbm_node & a, const vbm_node & b) {
    return a.ne[0] == b.ne[0] && a.ne[1] == b.ne[1] && a.ne[2] == b.ne[2] && a.ne[3] == b.ne[3];
}

float param_f32(const vbm_node & t, int i) {
    float v;
    std::memcpy(&v, &t.op_params[i], sizeof(v));
    return v;
}

// ---------------------------------------------------------------------------------------------
// supports_op: nullptr when the node can run here, else the reason it cannot
// ---------------------------------------------------------------------------------------------

const char * check_mul_mat_id(const vbm_node & t) {
    const vbm_node * as = t.src[0], * b = t.src[1], * ids = t.src[2];
    if (!as || !b || !ids) return "MUL_MAT_ID needs as, b and ids";
    if (!shape_valid(*as) || !shape_valid(*b) || !shape_valid(*ids) || !shape_valid(t)) return "bad tensor shape or type";
    if (as->type != VBM_TYPE_MXFP4 && as->type != VBM_TYPE_Q8_0) return "expert weights must be MXFP4 or Q8_0";
    if (as->ne[0] % 64 != 0 || as->ne[1] % 32 != 0 || as->ne[2] > 1024 || as->ne[3] != 1)
        return "expert tensor must be [k % 64, rows % 32, n_as <= 1024, 1]";
    if (ids->type != VBM_TYPE_I32 || ids->ne[2] != 1 || ids->ne[3] != 1) return "ids must be I32 [n_ids, n_tokens]";
    if ((ids->ne[0] > 1 && ids->nb[0] != sizeof(int32_t)) || ids->nb[1] % sizeof(int32_t) != 0 ||
        (ids->ne[1] > 1 && ids->nb[1] < ids->ne[0] * sizeof(int32_t)))
        return "ids rows must be contiguous with a token stride of at least n_ids";
    const int64_t n_ids = ids->ne[0], n_tokens = ids->ne[1];
    if (b->ne[0] != as->ne[0] || (b->ne[1] != 1 && b->ne[1] != n_ids) || b->ne[2] != n_tokens || b->ne[3] != 1)
        return "b must be [k, 1 or n_ids, n_tokens, 1]";
    if (b->type == VBM_TYPE_F32) {
        int64_t stride = 0;
        if (!uniform_rows(*b, &stride) || !aligned_strides(*b)) return "F32 b rows must be contiguous and evenly spaced";
    } else if (b->type == VBM_TYPE_Q8_0) {
        if (!contiguous(*b)) return "Q8_0 b must be contiguous";
    } else {
        return "b must be F32 or Q8_0";
    }
    if (t.type != VBM_TYPE_F32 || t.ne[0] != as->ne[1] || t.ne[1] != n_ids || t.ne[2] != n_tokens || t.ne[3] != 1)
        return "dst must be F32 [rows, n_ids, n_tokens, 1]";
    if (!contiguous(t)) return "dst must be contiguous";
    return nullptr;
}

const char * check_add_id(const vbm_node & t) {
    const vbm_node * a = t.src[0], * bias = t.src[1], * ids = t.src[2];
    if (!a || !bias || !ids) return "ADD_ID needs a, bias and ids";
    if (!shape_valid(*a) || !shape_valid(*bias) || !shape_valid(*ids) || !shape_valid(t)) return "bad tensor shape or type";
    if (a->type != VBM_TYPE_F32 || bias->type != VBM_TYPE_F32 || t.type != VBM_TYPE_F32) return "ADD_ID is F32";
    if (ids->type != VBM_TYPE_I32 || ids->ne[0] != a->ne[1] || ids->ne[1] != a->ne[2] || ids->ne[2] != 1 || ids->ne[3] != 1)
        return "ids must be I32 [n_ids, n_tokens] matching a";
    if (a->ne[3] != 1 || !same_shape(*a, t)) return "dst must have a's shape [rows, n_ids, n_tokens, 1]";
    if (bias->ne[0] != a->ne[0] || bias->ne[2] != 1 || bias->ne[3] != 1) return "bias must be [rows, n_as]";
    if (!aligned_strides(*a) || !aligned_strides(t) || !aligned_strides(*bias) || !aligned_strides(*ids))
        return "strides must be multiples of 4 bytes";
    if (bias->nb[0] != sizeof(float)) return "bias rows must be contiguous";
    return nullptr;
}

const char * check_binary(const vbm_node & t) {
    const vbm_node * a = t.src[0], * b = t.src[1];
    if (!a || !b) return "binary op needs two operands";
    if (!shape_valid(*a) || !shape_valid(*b) || !shape_valid(t)) return "bad tensor shape or type";
    if (a->type != VBM_TYPE_F32 || b->type != VBM_TYPE_F32 || t.type != VBM_TYPE_F32) return "ADD / MUL are F32 here";
    if (!same_shape(*a, t)) return "dst must have src0's shape";
    for (int d = 0; d < 4; ++d)
        if (a->ne[d] % b->ne[d] != 0) return "src1 must repeat to src0's shape";
    if (!aligned_strides(*a) || !aligned_strides(*b) || !aligned_strides(t)) return "strides must be multiples of 4 bytes";
    return nullptr;
}

const char * check_cont(const vbm_node & t) {
    const vbm_node * a = t.src[0];
    if (!a) return "CONT needs a source";
    if (!shape_valid(*a) || !shape_valid(t)) return "bad tensor shape or type";
    if (a->type != VBM_TYPE_F32 || t.type != VBM_TYPE_F32) return "CONT is F32 here";
    if (nelements(*a) != nelements(t) || !contiguous(t)) return "dst must be contiguous with src's element count";
    if (!aligned_strides(*a) || !aligned_strides(t)) return "strides must be multiples of 4 bytes";
    return nullptr;
}

// ggml_cast / ggml_cpy between F32 and I32 into a contiguous dst with src's element count
// (src[1] of a ggml CPY node is its destination, itself for a cast: not read here).
const char * check_cpy(const vbm_node & t) {
    const vbm_node * a = t.src[0];
    if (!a) return "CPY needs a source";
    if (!shape_valid(*a) || !shape_valid(t)) return "bad tensor shape or type";
    if ((a->type != VBM_TYPE_F32 && a->type != VBM_TYPE_I32) || (t.type != VBM_TYPE_F32 && t.type != VBM_TYPE_I32))
        return "CPY converts between F32 and I32 here";
    if (nelements(*a) != nelements(t) || !contiguous(t)) return "dst must be contiguous with src's element count";
    if (!aligned_strides(*a) || !aligned_strides(t)) return "strides must be multiples of 4 bytes";
    return nullptr;
}

const char * check_glu(const vbm_node & t) {
    const vbm_node * a = t.src[0], * b = t.src[1];
    const int op = t.op_params[0];
    if (op != VBM_GLU_OP_SWIGLU && op != VBM_GLU_OP_SWIGLU_OAI) return "GLU op must be swiglu or swiglu_oai";
    if (!a || !shape_valid(*a) || !shape_valid(t) || (b && !shape_valid(*b))) return "bad tensor shape or type";
    int64_t s = 0;
    if (!uniform_rows(*a, &s) || !uniform_rows(t, &s) || (b && !uniform_rows(*b, &s)))
        return "GLU operands must be F32 with contiguous, evenly spaced rows";
    if (!aligned_strides(*a) || !aligned_strides(t) || (b && !aligned_strides(*b))) return "strides must be multiples of 4 bytes";
    const int64_t width = b ? a->ne[0] : a->ne[0] / 2;
    if ((!b && a->ne[0] % 2 != 0) || t.ne[0] != width || t.ne[1] != a->ne[1] || t.ne[2] != a->ne[2] || t.ne[3] != a->ne[3])
        return "dst must be [width, rows...] of the gate operand";
    if (b && !same_shape(*a, *b)) return "gate and up must have one shape";
    return nullptr;
}

// ggml_cuda_host_call_supported (hybrid-experts.patch:963-983): contiguous operands with host
// buffers for a call; same-shape contiguous F32 operands for a join.
const char * check_custom(const vbm_node & t) {
    const auto * call = static_cast<const vbm_host_call *>(t.extra);
    if (!call) return "CUSTOM node needs its vbm_host_call descriptor in extra";
    if (!shape_valid(t) || !contiguous(t)) return "host-call output must be contiguous";
    if (call->magic == VBM_HOST_JOIN_MAGIC) {
        const vbm_node * a = t.src[0], * b = t.src[1];
        if (!call->call) return "join descriptor names no call";
        if (!a || !b || t.type != VBM_TYPE_F32 || a->type != VBM_TYPE_F32 || b->type != VBM_TYPE_F32) return "join is F32 a + b";
        if (!shape_valid(*a) || !shape_valid(*b) || !contiguous(*a) || !contiguous(*b) || !same_shape(*a, t) ||
            !same_shape(*b, t))
            return "join operands must be contiguous with dst's shape";
        return nullptr;
    }
    if (call->magic != VBM_HOST_CALL_MAGIC) return "extra is not a host-call descriptor";
    if (!call->dst_host) return "host call has no output host buffer";
    for (int i = 0; i < VBM_NODE_MAX_SRC && t.src[i]; ++i) {
        if (!shape_valid(*t.src[i]) || !contiguous(*t.src[i])) return "host-call inputs must be contiguous";
        if (!call->src_host[i]) return "host call has no host buffer for an input";
    }
    if (call->miss_src > 0) {
        if (call->miss_src > VBM_NODE_MAX_SRC || !t.src[call->miss_src - 1] || t.src[call->miss_src - 1]->type != VBM_TYPE_I32)
            return "miss_src must name an I32 input";
    }
    return nullptr;
}

const char * why_unsupported(const vbm_node & t) {
    switch (t.op) {
        case VBM_NODE_NONE:
        case VBM_NODE_VIEW: return nullptr;
        case VBM_NODE_ADD:
        case VBM_NODE_MUL: return check_binary(t);
        case VBM_NODE_CONT: return check_cont(t);
        case VBM_NODE_MUL_MAT_ID: return check_mul_mat_id(t);
        case VBM_NODE_ADD_ID: return check_add_id(t);
        case VBM_NODE_GLU: return check_glu(t);
        case VBM_NODE_CUSTOM: return check_custom(t);
        case VBM_NODE_CPY: return check_cpy(t);
        default: return "op not handled by this library";
    }
}

// ---------------------------------------------------------------------------------------------
// compute_forward
// ---------------------------------------------------------------------------------------------

template <int OP>
void launch_elementwise(const vbm_node & dst, const vbm_node & a, const vbm_node * b, hipStream_t s) {
    const int64_t n = nelements(a);
    Strides sd = strides_of(dst.nb);
    if (OP == EW_COPY) {   // CONT: dst is contiguous over src's shape
        sd.nb[0] = sizeof(float);
        for (int d = 1; d < 4; ++d) sd.nb[d] = sd.nb[d - 1] * a.ne[d - 1];
    }
    const vbm_node & bb = b ? *b : a;
    hipLaunchKernelGGL(elementwise_kernel<OP>, dim3(grid_for(n)), dim3(256), 0, s, static_cast<char *>(dst.data), sd,
                       static_cast<const char *>(a.data), strides_of(a.nb), static_cast<const char *>(bb.data),
                       strides_of(bb.nb), dims_of(a.ne), dims_of(bb.ne), n);
    check_hip(hipGetLastError(), "elementwise launch");
}

void launch_convert(const vbm_node & dst, const vbm_node & a, hipStream_t s) {
    const int64_t n = nelements(a);
    hipLaunchKernelGGL(convert_kernel, dim3(grid_for(n)), dim3(256), 0, s, static_cast<char *>(dst.data),
                       strides_of(dst.nb), dims_of(dst.ne), dst.type == VBM_TYPE_I32 ? 1 : 0,
                       static_cast<const char *>(a.data), strides_of(a.nb), dims_of(a.ne), a.type == VBM_TYPE_I32 ? 1 : 0, n);
    check_hip(hipGetLastError(), "convert launch");
}

void forward_mul_mat_id(const vbm_node & t, int order, hipStream_t s) {
    const vbm_node & as = *t.src[0], & b = *t.src[1], & ids = *t.src[2];
    const auto * binding = static_cast<const vbm_expert_tensor *>(as.extra);
    require(binding != nullptr && binding->bank != nullptr, "MUL_MAT_ID expert tensor has no bank bound in extra");
    const vbm_bank & bank = *binding->bank;
    require(bank.type == as.type && bank.k == as.ne[0] && bank.rows == as.ne[1],
            "bound bank does not hold this expert tensor's type and shape");
    int64_t b_stride = bank.k;
    if (b.type == VBM_TYPE_F32) uniform_rows(b, &b_stride);
    const int64_t n_ids = ids.ne[0], n_tokens = ids.ne[1];
    const int64_t ids_stride = n_tokens > 1 ? static_cast<int64_t>(ids.nb[1] / sizeof(int32_t)) : n_ids;
    check_mul_mat_id_shape(bank, as.ne[2], b.ne[1], n_ids, n_tokens, ids_stride, order);
    const size_t bytes = mul_mat_id_scratch_bytes(bank, as.ne[2], b.ne[1], n_ids, n_tokens, order);
    mul_mat_id(&bank, binding->expert_to_slot, binding->expert_to_slot_host, as.ne[2], b.type, b.data, b.ne[1],
               static_cast<const int32_t *>(ids.data), n_ids, n_tokens, ids_stride, nullptr,
               static_cast<float *>(t.data), order, static_cast<uint8_t *>(stream_scratch(s, bytes)), bytes, s, b_stride);
}

void forward_add_id(const vbm_node & t, hipStream_t s) {
    const vbm_node & a = *t.src[0], & bias = *t.src[1], & ids = *t.src[2];
    const int64_t n = nelements(a);
    hipLaunchKernelGGL(add_id_kernel, dim3(grid_for(n)), dim3(256), 0, s, static_cast<char *>(t.data), strides_of(t.nb),
                       static_cast<const char *>(a.data), strides_of(a.nb), static_cast<const char *>(bias.data),
                       static_cast<int64_t>(bias.nb[1]), bias.ne[1], static_cast<const char *>(ids.data),
                       static_cast<int64_t>(ids.nb[0]), static_cast<int64_t>(ids.nb[1]), dims_of(a.ne), n);
    check_hip(hipGetLastError(), "add_id launch");
}

void forward_glu(const vbm_node & t, hipStream_t s) {
    const vbm_node & a = *t.src[0];
    const vbm_node * b = t.src[1];
    const bool swapped = t.op_params[1] != 0;
    const int64_t width = t.ne[0], rows = t.ne[1] * t.ne[2] * t.ne[3];
    int64_t sa = 0, sb = 0, sd = 0;
    uniform_rows(a, &sa);
    uniform_rows(t, &sd);
    const float * first = static_cast<const float *>(a.data);
    const float * second = first + width;
    if (b) {
        uniform_rows(*b, &sb);
        second = static_cast<const float *>(b->data);
    } else {
        sb = sa;
    }
    const float * gate = swapped ? second : first, * up = swapped ? first : second;
    const int64_t gs = swapped ? sb : sa, us = swapped ? sa : sb;
    const bool oai = t.op_params[0] == VBM_GLU_OP_SWIGLU_OAI;
    launch_glu(oai ? VBM_ACT_SWIGLU_OAI : VBM_ACT_SILU, gate, up, static_cast<float *>(t.data), rows, width, gs, us, sd,
               oai ? param_f32(t, 2) : 0.0f, oai ? param_f32(t, 3) : 0.0f, s);
}

void forward_custom(const vbm_node & t, int mode, hipStream_t s) {
    auto * call = static_cast<vbm_host_call *>(t.extra);
    vbm_status st;
    if (call->magic == VBM_HOST_JOIN_MAGIC) {
        st = vbm_host_join(call->call, static_cast<const float *>(t.src[0]->data), static_cast<const float *>(t.src[1]->data),
                           static_cast<float *>(t.data), nelements(t), s);
    } else {
        const void * srcs[VBM_NODE_MAX_SRC] = {};
        size_t sizes[VBM_NODE_MAX_SRC] = {};
        int n_src = 0;
        for (; n_src < VBM_NODE_MAX_SRC && t.src[n_src]; ++n_src) {
            srcs[n_src] = t.src[n_src]->data;
            sizes[n_src] = nbytes(*t.src[n_src]);
        }
        const vbm_node * miss = call->miss_src > 0 ? t.src[call->miss_src - 1] : nullptr;
        st = vbm_host_call_enqueue(call, srcs, sizes, n_src, t.data, nbytes(t),
                                   miss ? static_cast<const int32_t *>(miss->data) : nullptr, miss ? nelements(*miss) : 0,
                                   mode, s);
    }
    if (st != VBM_OK) fail(st, vbm_last_error());
}

void compute_forward(const vbm_node * node, const vbm_compute_params * params, hipStream_t s) {
    require(node != nullptr, "null node");
    const vbm_node & t = *node;
    if (const char * why = why_unsupported(t)) fail(VBM_ERR_UNSUPPORTED, why);
    if (t.op == VBM_NODE_NONE || t.op == VBM_NODE_VIEW) return;
    require(t.data != nullptr, "node has no data");
    for (int i = 0; i < VBM_NODE_MAX_SRC && t.src[i]; ++i)
        require(t.src[i]->data != nullptr || (t.op == VBM_NODE_MUL_MAT_ID && i == 0), "node source has no data");
    const int order = params ? params->order : VBM_ORDER_EXACT;
    const int mode = params ? params->host_call_mode : VBM_HOST_CALL_FUNC;
    switch (t.op) {
        case VBM_NODE_ADD: launch_elementwise<EW_ADD>(t, *t.src[0], t.src[1], s); break;
        case VBM_NODE_MUL: launch_elementwise<EW_MUL>(t, *t.src[0], t.src[1], s); break;
        case VBM_NODE_CONT: launch_elementwise<EW_COPY>(t, *t.src[0], nullptr, s); break;
        case VBM_NODE_MUL_MAT_ID: forward_mul_mat_id(t, order, s); break;
        case VBM_NODE_ADD_ID: forward_add_id(t, s); break;
        case VBM_NODE_GLU: forward_glu(t, s); break;
        case VBM_NODE_CUSTOM: forward_custom(t, mode, s); break;
        case VBM_NODE_CPY: launch_convert(t, *t.src[0], s); break;
        default: fail(VBM_ERR_UNSUPPORTED, "op not handled by this library");
    }
}

}  // namespace

extern "C" {

int vbm_node_supported(const vbm_node * node) {
    return node != nullptr && why_unsupported(*node) == nullptr ? 1 : 0;
}

vbm_status vbm_compute_forward(const vbm_node * node, const vbm_compute_params * params, void * stream) {
    return guarded([&] { compute_forward(node, params, as_stream(stream)); });
}

vbm_status vbm_graph_compute(const vbm_node * const * nodes, int64_t n_nodes, const vbm_compute_params * params,
                             void * stream) {
    return guarded([&] {
        require(nodes != nullptr && n_nodes >= 0, "null node list");
        for (int64_t i = 0; i < n_nodes; ++i) {
            try {
                compute_forward(nodes[i], params, as_stream(stream));
            } catch (const Error & e) {
                fail(e.status, "node " + std::to_string(i) + ": " + e.what());
            }
        }
    });
}

vbm_status vbm_add_id(float * y, const float * bias, int64_t n_as, const int32_t * ids, int64_t rows, int64_t n_ids,
                      int64_t n_tokens, int64_t ids_stride, void * stream) {
    return guarded([&] {
        require(y && bias && ids && rows > 0 && n_ids > 0 && n_tokens > 0 && n_as > 0 && ids_stride >= n_ids,
                "invalid add_id");
        const int64_t n = rows * n_ids * n_tokens;
        const Strides sy{{4, rows * 4, rows * n_ids * 4, rows * n_ids * n_tokens * 4}};
        hipLaunchKernelGGL(add_id_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), reinterpret_cast<char *>(y), sy,
                           reinterpret_cast<const char *>(y), sy, reinterpret_cast<const char *>(bias), rows * 4, n_as,
                           reinterpret_cast<const char *>(ids), int64_t(4), ids_stride * 4,
                           Dims{{rows, n_ids, n_tokens, 1}}, n);
        check_hip(hipGetLastError(), "add_id launch");
    });
}

}  // extern "C"
