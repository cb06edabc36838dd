// The bandwidth-bound row kernels, one wave64 per row (the row functions of rowops.h): embed,
// norm_add and score (the reference's kernels/src/main.rs:47-200).
#include <algorithm>
#include <stdexcept>
#include <string>

#include "rowops.h"

namespace jh {

// One wave a row, all in one round (a long input's rows are all in flight at once). Measured at
// 18379 rows: two or four rows a wave with every load issued first, or a grid-stride loop that
// loads the next row under the current one's arithmetic, were 10-30% slower; the plain copy
// kernel moving the same bytes reaches ~70% of the HBM peak at this size.
template <int NC>
__global__ __launch_bounds__(256) void embed_kernel(const uint32_t* ids, int n, const f16* table,
                                                    int vocab, int d, const float* gamma, float eps,
                                                    f16* x) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;  // whole waves
    embed_row<NC, false>(ids, row, table, vocab, d, gamma, eps, x, threadIdx.x & 63);
}

template <int NC>
__global__ __launch_bounds__(256) void norm_add_kernel(const f16* x, int n, int d,
                                                       const float* gamma, const float* add,
                                                       const int32_t* row_type, float eps,
                                                       f16* out, float* stats) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    norm_add_row<NC, false>(x, row, d, gamma, add, row_type, eps, out, stats, threadIdx.x & 63);
}

// Rows markers[i] of a (and of b, and of the statistics sa, when given) into row i of a_out
// (b_out, sa_out): the marker rows, compacted for the head's last row-wise steps.
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint4* a, const uint4* b,
                                                          const float2* sa, int n, int d,
                                                          const uint32_t* markers, int k,
                                                          uint4* a_out, uint4* b_out,
                                                          float2* sa_out) {
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (i >= k) return;
    const size_t r = min(markers[i], (uint32_t)(n - 1));  // the host checks markers < n
    const int chunks = d / 8, groups = d / 64;
    for (int c = lane; c < chunks; c += 64) {
        a_out[(size_t)i * chunks + c] = a[r * chunks + c];
        if (b) b_out[(size_t)i * chunks + c] = b[r * chunks + c];
    }
    if (sa && lane < groups) sa_out[(size_t)i * groups + lane] = sa[r * groups + lane];
}

template <int NC>
__global__ __launch_bounds__(256) void score_kernel(const f16* y, int n, int d, const f16* w,
                                                    float b, const uint32_t* markers, int k,
                                                    float* logits) {
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= k) return;
    score_row<NC>(y, n, d, w, b, markers, i, logits, threadIdx.x & 63);
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

#define JH_ROW_DISPATCH(KERNEL, N, ST, ...)                                                      \
    do {                                                                                         \
        const int nc = (d / 4 + 63) / 64;                                                        \
        const dim3 grid((unsigned)(((N) + 3) / 4));                                              \
        if (nc <= 1) hipLaunchKernelGGL(KERNEL<1>, grid, dim3(256), 0, ST, __VA_ARGS__);          \
        else if (nc <= 2) hipLaunchKernelGGL(KERNEL<2>, grid, dim3(256), 0, ST, __VA_ARGS__);     \
        else if (nc <= 3) hipLaunchKernelGGL(KERNEL<3>, grid, dim3(256), 0, ST, __VA_ARGS__);     \
        else if (nc <= 4) hipLaunchKernelGGL(KERNEL<4>, grid, dim3(256), 0, ST, __VA_ARGS__);     \
        else hipLaunchKernelGGL(KERNEL<16>, grid, dim3(256), 0, ST, __VA_ARGS__);                 \
    } while (0)

void embed_launch(const uint32_t* ids, int n, const jh_half* table, int vocab, int d,
                  const float* gamma, float eps, jh_half* x, hipStream_t st) {
    check_row("embed", n, d, table, x);
    if (!ids || !gamma || vocab <= 0 || ((uintptr_t)gamma % 16))
        throw std::runtime_error("embed: bad ids, gamma or vocab");
    JH_ROW_DISPATCH(embed_kernel, n, st, ids, n, (const f16*)table, vocab, d, gamma,
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
    JH_ROW_DISPATCH(norm_add_kernel, n, st, (const f16*)x, n, d, gamma, add,
                    row_type, eps, (f16*)out, stats);
    check_launch("norm_add");
}

void gather_rows_launch(const jh_half* a, const jh_half* b, const float* stats, int n, int d,
                        const uint32_t* markers, int k, jh_half* a_out, jh_half* b_out,
                        float* stats_out, hipStream_t st) {
    check_row("gather", n, d, a, a_out);
    if (k <= 0) return;
    if (!markers || (b && (!b_out || ((uintptr_t)b % 16) || ((uintptr_t)b_out % 16))) ||
        (stats && (!stats_out || ((uintptr_t)stats % 8) || ((uintptr_t)stats_out % 8))))
        throw std::runtime_error("gather: bad markers, rows or statistics");
    hipLaunchKernelGGL(gather_rows_kernel, dim3((k + 3) / 4), dim3(256), 0, st, (const uint4*)a,
                       (const uint4*)b, (const float2*)stats, n, d, markers, k, (uint4*)a_out,
                       (uint4*)b_out, (float2*)stats_out);
    check_launch("gather");
}

void score_launch(const jh_half* y, int n, int d, const jh_half* w, float b,
                  const uint32_t* markers, int k, float* logits, hipStream_t st) {
    check_row("score", n, d, y, w);
    if (k <= 0) return;  // no markers: nothing to score
    if (!logits || (!markers && k > n)) throw std::runtime_error("score: null logits, or k > n rows");
    JH_ROW_DISPATCH(score_kernel, k, st, (const f16*)y, n, d, (const f16*)w, b,
                    markers, k, logits);
    check_launch("score");
}

}  // namespace jh
