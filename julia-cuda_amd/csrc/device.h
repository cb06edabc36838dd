// Device-side building blocks shared by the gfx950 kernels: f16 vector types, the MFMA
// 16x16x32 f16 step, wave64 reductions, the GELU of the reference and the GEMM epilogue.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

typedef _Float16 f16;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace jh {

// D = A . B + C for a 16 x 16 output, K = 32. Lane l holds row/column (l % 16) of A/B and
// eight K values (the lane group l / 16 picks which eight; A and B use the same map, so any
// consistent permutation of K between the two operands gives the same result). The result
// lane l holds D[4 (l / 16) + i][l % 16], i = 0..3.
__device__ __forceinline__ floatx4 mfma16(half8 a, half8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// v & keep on all 128 bits (keep is 0 or all ones): a select without a branch.
__device__ __forceinline__ half8 mask16(half8 v, uint32_t keep) {
    uint32_t u[4];
    __builtin_memcpy(u, &v, 16);
#pragma unroll
    for (int i = 0; i < 4; i++) u[i] &= keep;
    __builtin_memcpy(&v, u, 16);
    return v;
}

// v from another lane of the same 16-lane row, by a DPP lane pattern (no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// gfx950's lane swaps, as (lane l's value, lane l ^ 16's value) and (l, l ^ 32) pairs in some
// order that is the same for both lanes of a pair: v_permlane16_swap exchanges the odd 16-lane
// rows of one operand with the even rows of the other, v_permlane32_swap the upper half of one
// with the lower half of the other; with both operands v, the two results hold v of the lower and
// of the upper partner. A symmetric reduction of the pair needs no lane select.
struct LanePair {
    float lo, hi;
};
__device__ __forceinline__ LanePair lane_pair16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ LanePair lane_pair32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
// 2^x by the hardware's v_exp_f32 alone: exact at 0 and -inf (-> 0); results below 2^-126 come
// out as zero rather than denormals, which a softmax weight never misses (exp2f adds a rescaling
// step for them around the same instruction).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float max_xor16(float v) { const LanePair p = lane_pair16(v); return fmaxf(p.lo, p.hi); }
__device__ __forceinline__ float max_xor32(float v) { const LanePair p = lane_pair32(v); return fmaxf(p.lo, p.hi); }
__device__ __forceinline__ float sum_xor16(float v) { const LanePair p = lane_pair16(v); return p.lo + p.hi; }
__device__ __forceinline__ float sum_xor32(float v) { const LanePair p = lane_pair32(v); return p.lo + p.hi; }

// The sum over each group of `W` consecutive lanes (W a power of two <= 64), to every lane, with
// no LDS round trip. Within 16 lanes by DPP: quad_perm [1,0,3,2] and [2,3,0,1] (the quad's sum in
// every lane), the half-row mirror (lane i <- 7 - i: the other quad of 8), the row mirror
// (i <- 15 - i: the other 8 of 16); then the lane swaps. Every lane of a group gets the same bits
// (each step adds the same two values in either order).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "group width");
    if (W >= 2) v += dpp_move<0xB1>(v);
    if (W >= 4) v += dpp_move<0x4E>(v);
    if (W >= 8) v += dpp_move<0x141>(v);
    if (W >= 16) v += dpp_move<0x140>(v);
    if (W >= 32) v = sum_xor16(v);
    if (W >= 64) v = sum_xor32(v);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

// GELU(x) = x Phi(x), with erf(x / sqrt 2) from Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7),
// the approximation the reference uses (kernels/src/gemm.rs:139-150): t = 1 / (1 + p |x| / sqrt 2)
// with p = 0.3275911, and 1 - Phi(|x|) = poly(t) exp(-x^2 / 2) / 2.
__device__ __forceinline__ float gelu(float x) {
    const float p = 0.3275911f * 0.70710678118654752f;
    // the hardware reciprocal (1 ulp) in place of a correctly rounded division: the formula's own
    // error is 1.5e-7
    float t = __builtin_amdgcn_rcpf(1.0f + p * fabsf(x));
    // q = poly(t) exp(-x^2 / 2) / 2 with the polynomial's coefficients halved and exp(-x^2 / 2)
    // as exp2(x^2 (-log2(e) / 2)): halving is exact and commutes with rounding, and __expf is
    // the hardware exp2 of its argument times log2(e), so these are the values of
    // 0.5 poly __expf(-0.5 x x) bit for bit, with two multiplies fewer.
    const float hpoly = ((((0.5f * 1.061405429f * t - 0.5f * 1.453152027f) * t + 0.5f * 1.421413741f) * t -
                          0.5f * 0.284496736f) * t + 0.5f * 0.254829592f) * t;
    const float q = hpoly * __builtin_amdgcn_exp2f((x * x) * (-0.5f * 1.4426950408889634f));
    return x * (x >= 0.0f ? 1.0f - q : q);
}

// ---- hand-offs between blocks on different XCDs -------------------------------------------------
// The eight XCDs each have their own L2, which is not coherent with the others within a kernel.
// A general release (an agent-scope release fence) writes back the whole L2, which costs tens
// of microseconds per call here, and a general acquire invalidates it, which throws away what
// other blocks share through it. Data that another block reads in the same kernel (split-K and
// key-range partials, the layer kernel's phase outputs) is therefore stored AND loaded with
// agent-scope (device-coherent) accesses: the release is only "my stores have completed"
// (release_wait), and the reader needs no cache maintenance at all.
__device__ __forceinline__ void release_wait() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);  // every outstanding memory operation of this wave is done
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ void xstore64(void* p, uint64_t v) {
    __hip_atomic_store((uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 4-byte store, device-coherent when XG.
template <bool XG>
__device__ __forceinline__ void store4(void* p, half2 v) {
    if (XG) {
        uint32_t u;
        __builtin_memcpy(&u, &v, 4);
        __hip_atomic_store((uint32_t*)p, u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        *(half2*)p = v;
    }
}

// 8-byte stores, device-coherent when XG (the data is read by another block in this kernel).
template <bool XG>
__device__ __forceinline__ void store8(void* p, half4 v) {
    if (XG) {
        uint64_t u;
        __builtin_memcpy(&u, &v, 8);
        xstore64(p, u);
    } else {
        *(half4*)p = v;
    }
}

template <bool XG>
__device__ __forceinline__ void store8(void* p, float2 v) {
    if (XG) {
        uint64_t u;
        __builtin_memcpy(&u, &v, 8);
        xstore64(p, u);
    } else {
        *(float2*)p = v;
    }
}

template <bool XG>
__device__ __forceinline__ void store16(void* p, half8 v) {
    if (XG) {
        uint64_t u[2];
        __builtin_memcpy(u, &v, 16);
        xstore64(p, u[0]);
        xstore64((char*)p + 8, u[1]);
    } else {
        *(half8*)p = v;
    }
}

// Device-coherent loads for data another block wrote in this kernel: they fetch from the
// coherence point instead of a possibly stale L1/L2 line, so readers need no cache
// invalidation (which would also throw away the weights other blocks share through L2).
__device__ __forceinline__ uint64_t xload64(const void* p) {
    return __hip_atomic_load((uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool XG>
__device__ __forceinline__ half8 load16h(const f16* p) {
    if (XG) {
        const uint64_t u[2] = {xload64(p), xload64(p + 4)};
        half8 v;
        __builtin_memcpy(&v, u, 16);
        return v;
    }
    return *(const half8*)p;
}

template <bool XG>
__device__ __forceinline__ half4 load8h(const f16* p) {
    if (XG) {
        const uint64_t u = xload64(p);
        half4 v;
        __builtin_memcpy(&v, &u, 8);
        return v;
    }
    return *(const half4*)p;
}

template <bool XG>
__device__ __forceinline__ float2 load8f(const float* p) {
    if (XG) {
        const uint64_t u = xload64(p);
        float2 v;
        __builtin_memcpy(&v, &u, 8);
        return v;
    }
    return *(const float2*)p;
}

__device__ __forceinline__ float xload32(const float* p) {
    return __uint_as_float(__hip_atomic_load((uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

__device__ __forceinline__ void xstore32(float* p, float v) {
    __hip_atomic_store((uint32_t*)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Raw buffer access (gfx9 buffer descriptor: base, byte size, no stride): reads past `bytes`
// return zeros. With XG the 16-byte load is device-coherent (sc1), like xload64 but in one
// instruction.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

template <bool XG>
__device__ __forceinline__ half8 bload16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, XG ? 16 : 0));
}

// 16-byte buffer store at byte_off; with XG device-coherent (sc1) in one instruction, where a
// coherent global store takes two 8-byte ones.
template <bool XG>
__device__ __forceinline__ void bstore16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, half8 v) {
    typedef int int4_t __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(int4_t, v), r, byte_off, 0, XG ? 16 : 0);
}

// The same for four floats, device-coherent (the split-K partials: one 16-byte operation where a
// coherent global access takes two 8-byte atomics; measured 128 x 128 tiles at 512 rows, split
// 2 / 4 ways: 13.5 / 15.3 µs with the atomics, 11.1 / 11.5 with these).
__device__ __forceinline__ void bstore16f(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float4 v) {
    bstore16<true>(r, byte_off, __builtin_bit_cast(half8, v));
}

__device__ __forceinline__ float4 bload16f(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(float4, bload16<true>(r, byte_off));
}

// s_waitcnt lgkmcnt(0) alone: this wave's LDS (and scalar memory) operations are done; vector
// memory operations (loads, stores) may still be in flight.
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// s_waitcnt with vmcnt = n (n < 64) and no wait on the other counters (gfx9 encoding:
// vmcnt[3:0] in bits 3:0 and vmcnt[5:4] in bits 15:14, expcnt in 6:4, lgkmcnt in 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// gfx950's direct global -> LDS load: each lane's 16 bytes at `src` land at LDS `base` + 16 lane
// (base is wave-uniform). Counted like any vector load: s_waitcnt vmcnt covers it. XG: the read
// is device-coherent (sc1), for data another block wrote in this kernel.
template <bool XG = false>
__device__ __forceinline__ void lds_dma16(const void* src, void* base) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)base, 16, 0,
                                     XG ? 16 : 0);
}

// The same through a buffer descriptor: the lane's 16 bytes at byte `voff` of `r` (zeros past its
// size, with no memory access). The address is the descriptor (scalar) plus a 32-bit lane
// offset: no 64-bit address arithmetic per lane and copy.
// soff: a wave-uniform byte offset added to every lane's (a scalar operand).
template <bool XG = false>
__device__ __forceinline__ void lds_bdma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, void* base,
                                           uint32_t soff = 0) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)base, 16,
                                             voff, soff, 0, XG ? 16 : 0);
}

// gfx950's transposing LDS read (ds_read_b64_tr_b16): within each 16-lane group, lane i receives
// element i % 4 of the 8 bytes lanes 4 j + i / 4 address, as its element j (j < 4). Loading a
// row-major [key][d] tile this way hands a lane 4 consecutive keys of one d column.
__device__ __forceinline__ half4 lds_read_tr16(const void* p) {
    typedef short short4_t __attribute__((ext_vector_type(4)));
    const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) short4_t*)p);
    return __builtin_bit_cast(half4, v);
}

__device__ __forceinline__ uint32_t atomic_add_agent(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void atomic_store_agent(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t atomic_load_agent(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Blocks are dispatched to the XCDs round-robin (block b to XCD b % 8). This maps block b to a
// task index so that each XCD gets one contiguous run of the T tasks: consecutive tasks share a
// weight tile, so each weight tile is fetched into (mostly) one XCD's L2.
__device__ __forceinline__ int xcd_task(int b, int T) {
    const int x = b & 7, j = b >> 3, q = T >> 3, r = T & 7;
    return x * q + (x < r ? x : r) + j;
}

// ---- the GEMM epilogue ------------------------------------------------------------------------
// One thread's share of an output tile: 8 values of row `row`, columns gcol + c0 + e (lo) and
// gcol + 32 + c0 + e (hi), e < 4, where gcol is a multiple of 64 (the tile's 64-column group
// `grp`) and c0 a multiple of 4 below 32. The 8 threads sharing a row are 8 consecutive lanes
// (lane % 8 = c0 / 4), which the statistics reduce over. `valid` is row < m; every thread calls
// this (the reductions need the whole group).
//
// Order as the reference's gemm_tile (kernels/src/main.rs:931-1038): LayerNorm from the input
// statistics, bias, ReLU, GELU, RoPE, then GeGLU or the store with the residual and the output
// statistics of the stored f16 values. XG: the input statistics are read device-coherent (the
// persistent layer kernel, where other blocks of the same kernel wrote them).
//
// The outputs (and output statistics) are stored device-coherent on every path, written through
// the XCD's L2. In the persistent kernel other blocks read them in the same launch; between
// per-step kernels, a kernel's end has to write back the dirty lines its stores leave in its
// XCD's L2 before the next kernel, on all eight XCDs, may read them. Measured on the 293-token
// forward (same box, interleaved runs): 0.675 -> 0.655 ms a request. (The same for the attention
// and row kernels' outputs gained nothing more.)
//
// Everything the epilogue reads besides the accumulator (statistics, colsum, bias, the RoPE
// table, the residual) is loaded by epi_load_* when the tile starts, so those loads overlap the
// operand loads instead of costing dependent round trips after the K loop. The loads are
// unconditional (rows past m read row m - 1, never stored) and masked in epi_apply: a guarded
// load is a branch, where the compiler waits for every outstanding load.

// Statistics slots one lane of a row's 8-lane group prefetches: j and j + 8 (j = lane % 8), all
// of a row with k <= 1024; epi_apply loads the rest of a wider row itself.
constexpr int EPI_PRE_SLOTS = 2;

struct EpiCol {  // per column: colsum (LN), bias and the score's weights, lo and hi halves
    float4 cs[2], bs[2];
    half4 sw[2];
};

// The source row of output row r (r < m): rows[r] with a gather (clamped to the source's rows).
// (A compile-time choice: a load under a run-time branch would make the compiler wait for every
// load issued before it.)
template <int EPI>
__device__ __forceinline__ int src_row(const GemmParams& p, int r) {
    return (EPI & EPI_GATHER) ? (int)min(p.rows[r], (uint32_t)(p.src_m - 1)) : r;
}
struct EpiRow {  // per row: statistics slots, position (as loaded), RoPE (cos, sin) pairs,
    float2 st[EPI_PRE_SLOTS];  // residual lo, hi
    int pos;
    float4 rt[2];
    half4 rl, rh;
};

template <int EPI>
__device__ __forceinline__ void epi_load_col(const GemmParams& p, int grp, int c0, EpiCol& e) {
    const int gcol = grp * 64;
    if (EPI & EPI_LN) {
        e.cs[0] = *(const float4*)(p.colsum + gcol + c0);
        e.cs[1] = *(const float4*)(p.colsum + gcol + 32 + c0);
    }
    if (EPI & EPI_BIAS) {
        e.bs[0] = *(const float4*)(p.bias + gcol + c0);
        e.bs[1] = *(const float4*)(p.bias + gcol + 32 + c0);
    }
    if (EPI & EPI_SCORE) {
        e.sw[0] = *(const half4*)((const f16*)p.score_w + gcol + c0);
        e.sw[1] = *(const half4*)((const f16*)p.score_w + gcol + 32 + c0);
    }
}

// XS: the statistics are read device-coherent; XR: the residual rows are.
template <int EPI, bool XS, bool XR = XS>
__device__ __forceinline__ void epi_load_row(const GemmParams& p, int row, int grp, int c0,
                                             EpiRow& e) {
    const int r = min(row, p.m - 1), rs = src_row<EPI>(p, r);
    if (EPI & EPI_LN) {
        const int slots = p.k >> 6, j = c0 >> 2;
        const float* st = p.stats_in + (size_t)rs * slots * 2;
#pragma unroll
        for (int i = 0; i < EPI_PRE_SLOTS; i++) e.st[i] = load8f<XS>(st + 2 * min(j + 8 * i, slots - 1));
    }
    if (EPI & EPI_ROPE) {
        // An unconditional load (from the table itself when there are no positions): a load
        // under a branch leaves the compiler unsure where it is in the load order, and the
        // table loads that wait for it would then wait for every load issued before them.
        // The choice between it and the row waits for the load: epi_load_rope makes it.
        e.pos = *(const int*)(p.pos ? (const void*)(p.pos + r) : (const void*)p.rope);
    }
    if ((EPI & EPI_RES) && !(EPI & EPI_GEGLU)) {
        const f16* x = (const f16*)(p.res ? p.res : p.c) + (size_t)(p.res ? rs : r) * p.n + grp * 64 + c0;
        e.rl = load8h<XR>(x);
        e.rh = load8h<XR>(x + 32);
    }
}

// The RoPE table row of output row `row`'s position (e.pos, loaded by epi_load_row): a separate
// step, so that a tile issues every row's position load before any table load (which waits for
// its position).
template <int EPI>
__device__ __forceinline__ void epi_load_rope(const GemmParams& p, int row, int c0, EpiRow& e) {
    if (EPI & EPI_ROPE) {
        const int pos = min(max(p.pos ? e.pos : min(row, p.m - 1), 0), p.rope_rows - 1);
        const float4* t = (const float4*)(p.rope + ((size_t)pos * 32 + c0) * 2);
        e.rt[0] = t[0];
        e.rt[1] = t[1];
    }
}

template <int EPI, bool XG = false>
__device__ __forceinline__ void epi_apply(const GemmParams& p, int row, int grp, int c0, float* v,
                                          bool valid, const EpiCol& ec, const EpiRow& er) {
    const int gcol = grp * 64;
    if (EPI & EPI_LN) {
        const int slots = p.k >> 6, j = c0 >> 2;
        float S = 0.0f, Q = 0.0f;
#pragma unroll
        for (int i = 0; i < EPI_PRE_SLOTS; i++)
            if (j + 8 * i < slots) S += er.st[i].x, Q += er.st[i].y;
        const float* st = p.stats_in + (size_t)src_row<EPI>(p, min(row, p.m - 1)) * slots * 2;
        for (int s = j + 8 * EPI_PRE_SLOTS; s < slots; s += 8) {  // rows wider than 1024
            const float2 sq = load8f<XG>(st + 2 * s);
            S += sq.x, Q += sq.y;
        }
        S = group_sum<8>(S);
        Q = group_sum<8>(Q);
        const float mean = S / (float)p.k;
        const float var = fmaxf(Q / (float)p.k - mean * mean, 0.0f);
        const float rs = 1.0f / sqrtf(var + p.eps);
        const float cs[8] = {ec.cs[0].x, ec.cs[0].y, ec.cs[0].z, ec.cs[0].w,
                             ec.cs[1].x, ec.cs[1].y, ec.cs[1].z, ec.cs[1].w};
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = rs * (v[e] - mean * cs[e]);
    }
    if (EPI & EPI_BIAS) {
        const float bs[8] = {ec.bs[0].x, ec.bs[0].y, ec.bs[0].z, ec.bs[0].w,
                             ec.bs[1].x, ec.bs[1].y, ec.bs[1].z, ec.bs[1].w};
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] += bs[e];
    }
    if (EPI & EPI_RELU) {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = fmaxf(v[e], 0.0f);
    }
    if (EPI & EPI_GELU) {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = gelu(v[e]);
    }
    if (EPI & EPI_ROPE) {
        // q and k heads: columns i and i + 32 of a head are the rotate-half pair of dimension i.
        if (gcol < p.rope_cols) {
            const float4 t0 = er.rt[0], t1 = er.rt[1];
            const float cs[4] = {t0.x, t0.z, t1.x, t1.z}, sn[4] = {t0.y, t0.w, t1.y, t1.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float x1 = v[e], x2 = v[4 + e];
                v[e] = x1 * cs[e] - x2 * sn[e];
                v[4 + e] = x2 * cs[e] + x1 * sn[e];
            }
        }
    }
    if (EPI & EPI_GEGLU) {
        // Packed rows 64 grp + e are the input of output column 32 grp + e, + 32 its gate.
        if (valid) {
            half4 o;
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = (f16)(gelu(v[e]) * v[4 + e]);
            store8<true>((f16*)p.c + (size_t)row * (p.n >> 1) + grp * 32 + c0, o);
        }
    } else {
        half4 lo, hi;
        f16* out = (f16*)p.c + (size_t)row * p.n + gcol + c0;
        if (EPI & EPI_RES) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                v[e] += (float)er.rl[e];
                v[4 + e] += (float)er.rh[e];
            }
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            lo[e] = (f16)v[e];
            hi[e] = (f16)v[4 + e];
        }
        if (EPI & EPI_SCORE) {  // the row's partial dot product over the tile's 64 columns
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++)
                s += (float)lo[e] * (float)ec.sw[0][e] + (float)hi[e] * (float)ec.sw[1][e];
            s = group_sum<8>(s);
            if (valid && (threadIdx.x & 7) == 0) xstore32(p.ws + (size_t)row * p.tiles_n + grp, s);
        } else if (valid) {
            store8<true>(out, lo);
            store8<true>(out + 32, hi);
        }
        if (EPI & EPI_STATS) {
            float s = 0.0f, q = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float a = (float)lo[e], b = (float)hi[e];
                s += a + b;
                q += a * a + b * b;
            }
            s = group_sum<8>(s);
            q = group_sum<8>(q);
            if (valid && (threadIdx.x & 7) == 0) {
                store8<true>(p.stats_out + ((size_t)row * (p.n >> 6) + grp) * 2, make_float2(s, q));
            }
        }
    }
}

}  // namespace jh
