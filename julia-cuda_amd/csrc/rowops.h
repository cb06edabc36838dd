// One row of the bandwidth-bound row operations, as device functions for a wave64: embed
// (table gather + LayerNorm), norm_add (the head's input: LayerNorm + type embedding, and the
// row statistics) and score (the scorer's last linear on a marker row). The reference's are
// kernels/src/main.rs:47-200 (one 32-lane warp per row, D fixed at 384); here D is any multiple
// of 64 up to 256 NC and a lane takes 4 f16 (8 bytes) at a time, 64 lanes covering 512
// contiguous bytes per step. The row kernels (rowops.hip) and the whole-model persistent kernel
// (layer.hip) share them. XG: the outputs are stored device-coherent (the persistent kernel's
// other blocks read them in the same launch).
#pragma once

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

// x[row] = LN(v) . gamma, rounded to f16, for v = table row ids[row] loaded by load_row
// (kernels/src/main.rs:47-103).
template <int NC, bool XG>
__device__ __forceinline__ void embed_store(const float (&v)[NC][4], int row, int d,
                                            const float* gamma, float eps, f16* x, int lane) {
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
            store8<XG>(x + (size_t)row * d + 4 * c, o);
        }
    }
}

// The table row of token id (clamped: the host checks ids < vocab).
__device__ __forceinline__ const f16* embed_src(const f16* table, uint32_t id, int vocab, int d) {
    return table + (size_t)min(id, (uint32_t)(vocab - 1)) * d;
}

// x[row] = LN(table[ids[row]]) . gamma, rounded to f16 (kernels/src/main.rs:47-103).
template <int NC, bool XG>
__device__ __forceinline__ void embed_row(const uint32_t* ids, int row, const f16* table, int vocab,
                                          int d, const float* gamma, float eps, f16* x, int lane) {
    float v[NC][4];
    load_row<NC>(embed_src(table, ids[row], vocab, d), d, lane, v);
    embed_store<NC, XG>(v, row, d, gamma, eps, x, lane);
}

// out[row] = LN(v) . gamma + add (+ row_type[row] * d when row_type is given), v = x[row] loaded
// by load_row; stats[row][g] = (sum, sum of squares) of the stored f16 values of 64-column group
// g (chunks 16 g .. 16 g + 15: lanes 16 (g % 4) .. + 15 of step g / 4)
// (kernels/src/main.rs:108-176).
template <int NC, bool XG>
__device__ __forceinline__ void norm_add_store(const float (&v)[NC][4], int row, int d,
                                               const float* gamma, const float* add,
                                               const int32_t* row_type, float eps, f16* out,
                                               float* stats, int lane) {
    if (row_type) add += (size_t)row_type[row] * d;
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
            store8<XG>(out + (size_t)row * d + 4 * c, o);
        }
        s = group_sum<16>(s);
        q = group_sum<16>(q);
        if ((lane & 15) == 0 && c < (d >> 2))
            store8<XG>(stats + ((size_t)row * (d >> 6) + (c >> 4)) * 2, make_float2(s, q));
    }
}

// norm_add_store of row `row` of x.
template <int NC, bool XG>
__device__ __forceinline__ void norm_add_row(const f16* x, int row, int d, const float* gamma,
                                             const float* add, const int32_t* row_type, float eps,
                                             f16* out, float* stats, int lane) {
    float v[NC][4];
    load_row<NC>(x + (size_t)row * d, d, lane, v);
    norm_add_store<NC, XG>(v, row, d, gamma, add, row_type, eps, out, stats, lane);
}

// logits[i] = v . u + b for a loaded row v and the loaded weights u (kernels/src/main.rs:180-200).
template <int NC>
__device__ __forceinline__ void score_dot(const float (&v)[NC][4], const float (&u)[NC][4], float b,
                                          int i, float* logits, int lane) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NC; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc += v[j][e] * u[j][e];
    acc = wave_sum(acc);
    if (lane == 0) logits[i] = acc + b;
}

// logits[i] = y[markers[i]] . w + b (kernels/src/main.rs:180-200); markers null: row i.
template <int NC>
__device__ __forceinline__ void score_row(const f16* y, int n, int d, const f16* w, float b,
                                          const uint32_t* markers, int i, float* logits, int lane) {
    // (the host checks markers < n)
    const uint32_t r = markers ? min(markers[i], (uint32_t)(n - 1)) : (uint32_t)i;
    float v[NC][4], u[NC][4];
    load_row<NC>(y + (size_t)r * d, d, lane, v);
    load_row<NC>(w, d, lane, u);
    score_dot<NC>(v, u, b, i, logits, lane);
}

}  // namespace jh
