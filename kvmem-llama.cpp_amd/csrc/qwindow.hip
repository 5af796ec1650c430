// Per-token query window on the device: the query rows the per-token max
// scorer reads, kept where the reference keeps only their sum.
//
// The reference harvests the pre-RoPE, post-q_norm query rows of the query
// span per layer into q_sum_ / q_count_ (harvest_capture('q') and
// harvest_from_host('q'), src/adapter/llama-memory-kvmem.cpp:2157-2172,
// 2206-2219; the strided view is read as ggml lays Qcur out: element (d, h,
// t) at d*nb0 + h*nb1 + t*nb2, bytes_to_f32_token_major :2066-2090).  Here
// the rows themselves are kept, widened to f32 exactly, in a ring of rows
// per layer; at preview they are gathered in token order, either narrowed
// for the MFMA scorer or summed (kvmem_hip_q_accumulate) for the mean-K
// scorer, which then matches the reference's sums bit for bit.
#include "kvmem_internal.hpp"

namespace kvmem_hip {

template <typename QT>
__device__ inline float q_elem(const uint8_t *p) {
    return static_cast<float>(*reinterpret_cast<const QT *>(p));
}

// grid (n, ceil(E / 256)): pair i = (token in the view, window row).
template <typename QT>
__global__ __launch_bounds__(256) void qwin_write_kernel(const uint8_t *q, uint64_t nb0, uint64_t nb1,
                                                         uint64_t nb2, uint32_t head_dim, uint32_t E,
                                                         const uint32_t *pairs, float *window) {
    const uint32_t i = blockIdx.x;
    const uint32_t e = blockIdx.y * 256u + threadIdx.x;
    if (e >= E) {
        return;
    }
    const uint32_t t = pairs[2 * i];
    const uint32_t r = pairs[2 * i + 1];
    const uint32_t h = e / head_dim;
    const uint32_t d = e - h * head_dim;
    window[static_cast<uint64_t>(r) * E + e] = q_elem<QT>(q + d * nb0 + h * nb1 + t * nb2);
}

// f32 -> bf16, round to nearest even (NaN stays a quiet NaN).
__device__ inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return static_cast<uint16_t>((u >> 16) | 0x40u);
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// grid (n, L): out[l][i][:] = window[l][rows[i]][:] in the output type.
__global__ __launch_bounds__(256) void qwin_gather_kernel(const float *window, uint32_t cap, uint32_t E,
                                                          const uint8_t *rows_dev, ArgTables rows_args,
                                                          uint32_t n, int out_type, uint8_t *out) {
    const uint32_t i = blockIdx.x;
    const uint32_t l = blockIdx.y;
    const uint32_t row = tab_read<uint32_t>(rows_dev, rows_args, 4u * i);
    const float *src = window + (static_cast<uint64_t>(l) * cap + row) * E;
    const uint64_t o = (static_cast<uint64_t>(l) * n + i) * E;
    for (uint32_t e = threadIdx.x; e < E; e += 256u) {
        const float v = src[e];
        if (out_type == KVMEM_TYPE_BF16) {
            reinterpret_cast<uint16_t *>(out)[o + e] = f32_to_bf16_rne(v);
        } else if (out_type == KVMEM_TYPE_F16) {
            reinterpret_cast<_Float16 *>(out)[o + e] = static_cast<_Float16>(v);
        } else {
            reinterpret_cast<float *>(out)[o + e] = v;
        }
    }
}

bool load_qwindow_kernels() {
    return load_kernel_object(&qwin_gather_kernel);
}

}  // namespace kvmem_hip

using namespace kvmem_hip;

extern "C" {

int kvmem_hip_q_window_write(kvmem_hip_ctx *ctx, const void *q, int32_t q_type, uint32_t n_head,
                             uint32_t head_dim, size_t nb0, size_t nb1, size_t nb2,
                             const uint32_t *tokens, const uint32_t *rows, uint32_t n, float *window,
                             uint32_t capacity) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n == 0) {
        return KVMEM_HIP_OK;
    }
    if (!q || !tokens || !rows || !window || n_head == 0 || head_dim == 0) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "q_window_write: null argument or empty geometry");
    }
    if (q_type != KVMEM_TYPE_F32 && q_type != KVMEM_TYPE_F16 && q_type != KVMEM_TYPE_BF16) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "q_window_write: query must be F32, F16 or BF16");
    }
    const size_t esz = q_type == KVMEM_TYPE_F32 ? 4 : 2;
    if (nb0 % esz || nb1 % esz || nb2 % esz || (reinterpret_cast<uintptr_t>(q) % esz) ||
        (reinterpret_cast<uintptr_t>(window) & 3u)) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "q_window_write: strides must be multiples of the element size");
    }
    const uint32_t E = n_head * head_dim;
    std::vector<uint32_t> pairs(2 * static_cast<size_t>(n));
    std::vector<uint8_t> seen(capacity, 0);
    for (uint32_t i = 0; i < n; ++i) {
        if (rows[i] >= capacity) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "q_window_write: row beyond the window's capacity");
        }
        if (seen[rows[i]]) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "q_window_write: a row is written twice");
        }
        seen[rows[i]] = 1;
        pairs[2 * i] = tokens[i];
        pairs[2 * i + 1] = rows[i];
    }
    (void) hipSetDevice(ctx->device);
    const uint32_t *dp = static_cast<const uint32_t *>(
        upload(ctx, pairs.data(), pairs.size() * sizeof(uint32_t), "q_window_write list"));
    if (!dp) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "q_window_write launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    const dim3 grid(n, (E + 255u) / 256u);
    const uint8_t *qb = static_cast<const uint8_t *>(q);
    if (q_type == KVMEM_TYPE_F32) {
        qwin_write_kernel<float><<<grid, 256, 0, ctx->stream>>>(qb, nb0, nb1, nb2, head_dim, E, dp, window);
    } else if (q_type == KVMEM_TYPE_F16) {
        qwin_write_kernel<_Float16><<<grid, 256, 0, ctx->stream>>>(qb, nb0, nb1, nb2, head_dim, E, dp, window);
    } else {
        qwin_write_kernel<__bf16><<<grid, 256, 0, ctx->stream>>>(qb, nb0, nb1, nb2, head_dim, E, dp, window);
    }
    return hip_ok(ctx, hipGetLastError(), "q_window_write launch") ? KVMEM_HIP_OK : KVMEM_HIP_ERR_RUNTIME;
}

int kvmem_hip_q_window_gather(kvmem_hip_ctx *ctx, const float *window, uint32_t n_layers,
                              uint32_t capacity, uint32_t n_embd_q, const uint32_t *rows, uint32_t n,
                              int32_t out_type, void *out) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n == 0 || n_layers == 0) {
        return KVMEM_HIP_OK;
    }
    if (!window || !rows || !out || n_embd_q == 0) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "q_window_gather: null argument");
    }
    if (out_type != KVMEM_TYPE_F32 && out_type != KVMEM_TYPE_F16 && out_type != KVMEM_TYPE_BF16) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "q_window_gather: output must be F32, F16 or BF16");
    }
    for (uint32_t i = 0; i < n; ++i) {
        if (rows[i] >= capacity) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "q_window_gather: row beyond the capacity");
        }
    }
    if (n_layers > 65535u) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "q_window_gather: too many layers");
    }
    (void) hipSetDevice(ctx->device);
    // the row list travels in the kernel arguments when it fits (768 rows)
    LaunchTables lt;
    if (!stage_tables(ctx, rows, sizeof(uint32_t) * n, lt, "q_window_gather rows")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "q_window_gather launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    qwin_gather_kernel<<<dim3(n, n_layers), 256, 0, ctx->stream>>>(window, capacity, n_embd_q, lt.dev, lt.args, n,
                                                                  out_type, static_cast<uint8_t *>(out));
    return hip_ok(ctx, hipGetLastError(), "q_window_gather launch") ? KVMEM_HIP_OK : KVMEM_HIP_ERR_RUNTIME;
}

}  // extern "C"
