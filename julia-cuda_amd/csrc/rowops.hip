// The bandwidth-bound row kernels, one wave64 per row: embed (table gather + LayerNorm),
// norm_add (the head's input: LayerNorm + type embedding, and the row statistics) and score
// (the scorer's last linear on the marker rows). The reference's are kernels/src/main.rs:47-200
// (one 32-lane warp per row, D fixed at 384); here D is any multiple of 64 and a lane takes
// 4 f16 (8 bytes) at a time, 64 lanes covering 512 contiguous bytes per step.
#include <algorithm>
#include <stdexcept>
#include <string>

#include "device.h"

namespace jh {

// Loads row `src` (d f16) as chunks c = lane + 64 j of 4 values, j < NC (chunks past d/4 are 0).
template <int NC>
__device__ __forceinline__ void load_row(const f16* src, int d, int lane, float (&v)[NC][4]) {
#pragma unroll
    for (int j = 0; j < NC; j++) {
        const int c = lane + 64 * j;
        if (c < (d >> 2)) {
            const half4 q = *(const half4*)(src + 4 * c);
#pragma unroll
            for (int e = 0; e < 4; e++) v[j][e] = (float)q[e];
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) v[j][e] = 0.0f;
        }
    }
}

// Two-pass LayerNorm statistics over d values (src/check.rs:62-83's emulation; the mean first,
// then the mean square deviation), as (mean, 1 / sqrt(var + eps)).
template <int NC>
__device__ __forceinline__ float2 ln_two_pass(const float (&v)[NC][4], int d, int lane, float eps) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NC; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) s += v[j][e];
    const float mean = wave_sum(s) / (float)d;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < NC; j++)
        if (lane + 64 * j < (d >> 2))
#pragma unroll
            for (int e = 0; e < 4; e++) q += (v[j][e] - mean) * (v[j][e] - mean);
    const float var = wave_sum(q) / (float)d;
    return make_float2(mean, 1.0f / sqrtf(var + eps));
}

template <int NC>
__global__ __launch_bounds__(256) void embed_kernel(const uint32_t* ids, int n, const f16* table,
                                                    int vocab, int d, const float* gamma, float eps,
                                                    f16* x) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= n) return;  // whole waves
    const uint32_t id = min(ids[row], (uint32_t)(vocab - 1));  // the host checks ids < vocab
    float v[NC][4];
    load_row<NC>(table + (size_t)id * d, d, lane, v);
    const float2 st = ln_two_pass<NC>(v, d, lane, eps);
#pragma unroll
    for (int j = 0; j < NC; j++) {
        const int c = lane + 64 * j;
        if (c < (d >> 2)) {
            const float4 gm = *(const float4*)(gamma + 4 * c);
            const float gs[4] = {gm.x, gm.y, gm.z, gm.w};
            half4 o;
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = (f16)((v[j][e] - st.x) * st.y * gs[e]);
            *(half4*)(x + (size_t)row * d + 4 * c) = o;
        }
    }
}

// out = LN(x) . gamma + add; stats[row][g] = (sum, sum of squares) of the stored f16 values of
// 64-column group g (chunks 16 g .. 16 g + 15: lanes 16 (g % 4) .. + 15 of step g / 4).
template <int NC>
__global__ __launch_bounds__(256) void norm_add_kernel(const f16* x, int n, int d,
                                                       const float* gamma, const float* add,
                                                       const int32_t* row_type, float eps,
                                                       f16* out, float* stats) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= n) return;
    if (row_type) add += (size_t)row_type[row] * d;
    float v[NC][4];
    load_row<NC>(x + (size_t)row * d, d, lane, v);
    const float2 st = ln_two_pass<NC>(v, d, lane, eps);
#pragma unroll
    for (int j = 0; j < NC; j++) {
        const int c = lane + 64 * j;
        float s = 0.0f, q = 0.0f;
        if (c < (d >> 2)) {
            const float4 gm = *(const float4*)(gamma + 4 * c);
            const float4 ad = *(const float4*)(add + 4 * c);
            const float gs[4] = {gm.x, gm.y, gm.z, gm.w}, as[4] = {ad.x, ad.y, ad.z, ad.w};
            half4 o;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                o[e] = (f16)((v[j][e] - st.x) * st.y * gs[e] + as[e]);
                const float y = (float)o[e];
                s += y;
                q += y * y;
            }
            *(half4*)(out + (size_t)row * d + 4 * c) = o;
        }
        s = group_sum<16>(s);
        q = group_sum<16>(q);
        if ((lane & 15) == 0 && c < (d >> 2))
            *(float2*)(stats + ((size_t)row * (d >> 6) + (c >> 4)) * 2) = make_float2(s, q);
    }
}

template <int NC>
__global__ __launch_bounds__(256) void score_kernel(const f16* y, int n, int d, const f16* w,
                                                    float b, const uint32_t* markers, int k,
                                                    float* logits) {
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (i >= k) return;
    const uint32_t r = min(markers[i], (uint32_t)(n - 1));  // the host checks markers < n
    float v[NC][4], u[NC][4];
    load_row<NC>(y + (size_t)r * d, d, lane, v);
    load_row<NC>(w, d, lane, u);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NC; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc += v[j][e] * u[j][e];
    acc = wave_sum(acc);
    if (lane == 0) logits[i] = acc + b;
}

// dst = src, 16 bytes per thread per step, grid-stride: the plain copy kernel the byte counters
// (rocprofv3 FETCH_SIZE / WRITE_SIZE) are calibrated against, and the achievable-bandwidth
// probe for the bandwidth-bound kernels.
__global__ __launch_bounds__(256) void stream_copy_kernel(const uint4* src, uint4* dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        dst[i] = src[i];
}

void stream_copy_launch(void* dst, const void* src, size_t bytes, hipStream_t st) {
    if (bytes % 16 || ((uintptr_t)dst % 16) || ((uintptr_t)src % 16))
        throw std::runtime_error("copy: 16-byte aligned buffers and sizes only");
    const size_t n = bytes / 16;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 8192);
    if (n) hipLaunchKernelGGL(stream_copy_kernel, dim3(blocks), dim3(256), 0, st, (const uint4*)src,
                              (uint4*)dst, n);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw std::runtime_error(std::string("copy: ") + hipGetErrorString(e));
}

namespace {

void check_row(const char* what, int n, int d, const void* a, const void* b) {
    if (n <= 0) throw std::runtime_error(std::string(what) + ": no rows");
    if (d <= 0 || d % 64 || d > 4096)
        throw std::runtime_error(std::string(what) + ": d = " + std::to_string(d) +
                                 " is not a multiple of 64 up to 4096");
    if (((uintptr_t)a % 16) || ((uintptr_t)b % 16))
        throw std::runtime_error(std::string(what) + ": buffers must be 16-byte aligned");
}

void check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace

#define JH_ROW_DISPATCH(KERNEL, GRID, ST, ...)                                                   \
    do {                                                                                         \
        const int nc = (d / 4 + 63) / 64;                                                        \
        if (nc <= 1) hipLaunchKernelGGL(KERNEL<1>, GRID, dim3(256), 0, ST, __VA_ARGS__);          \
        else if (nc <= 2) hipLaunchKernelGGL(KERNEL<2>, GRID, dim3(256), 0, ST, __VA_ARGS__);     \
        else if (nc <= 3) hipLaunchKernelGGL(KERNEL<3>, GRID, dim3(256), 0, ST, __VA_ARGS__);     \
        else if (nc <= 4) hipLaunchKernelGGL(KERNEL<4>, GRID, dim3(256), 0, ST, __VA_ARGS__);     \
        else hipLaunchKernelGGL(KERNEL<16>, GRID, dim3(256), 0, ST, __VA_ARGS__);                 \
    } while (0)

void embed_launch(const uint32_t* ids, int n, const jh_half* table, int vocab, int d,
                  const float* gamma, float eps, jh_half* x, hipStream_t st) {
    check_row("embed", n, d, table, x);
    if (!ids || !gamma || vocab <= 0 || ((uintptr_t)gamma % 16))
        throw std::runtime_error("embed: bad ids, gamma or vocab");
    JH_ROW_DISPATCH(embed_kernel, dim3((n + 3) / 4), st, ids, n, (const f16*)table, vocab, d, gamma,
                    eps, (f16*)x);
    check_launch("embed");
}

void norm_add_launch(const jh_half* x, int n, int d, const float* gamma, const float* add,
                     float eps, jh_half* out, float* stats, hipStream_t st,
                     const int32_t* row_type) {
    check_row("norm_add", n, d, x, out);
    if (!gamma || !add || !stats || ((uintptr_t)gamma % 16) || ((uintptr_t)add % 16) ||
        ((uintptr_t)stats % 8) || x == out)
        throw std::runtime_error("norm_add: bad gamma, add or stats, or out aliases x");
    JH_ROW_DISPATCH(norm_add_kernel, dim3((n + 3) / 4), st, (const f16*)x, n, d, gamma, add,
                    row_type, eps, (f16*)out, stats);
    check_launch("norm_add");
}

void score_launch(const jh_half* y, int n, int d, const jh_half* w, float b,
                  const uint32_t* markers, int k, float* logits, hipStream_t st) {
    check_row("score", n, d, y, w);
    if (k <= 0) return;  // no markers: nothing to score
    if (!markers || !logits) throw std::runtime_error("score: null markers or logits");
    JH_ROW_DISPATCH(score_kernel, dim3((k + 3) / 4), st, (const f16*)y, n, d, (const f16*)w, b,
                    markers, k, logits);
    check_launch("score");
}

}  // namespace jh
