// One output tile of the latency GEMM (BM = 16/32/64 rows x 64 columns), as a device function:
// the body of the per-GEMM `gemm_lat` kernels and a task of the persistent layer kernel, which
// pass their own LDS. See gemm.hip for the design.
#pragma once

#include "device.h"

namespace jh {

// LDS floats gemm_lat_tile<BM> needs: four waves' partial BM x 64 tiles, rows padded to 68.
template <int BM>
constexpr int lat_lds_floats() { return 4 * BM * 68; }

// Shared tail: each thread's 8 values (K fully summed within the block) -> the split-K
// reduction when the grid splits K -> the epilogue. Thread t owns row (pass * 32 + t / 8) of the
// tile and columns c0 = 4 (t % 8), c0 + 32 of 64-column group `grp`.
//
// Split-K (kernels/src/gemm.rs:355-433): every block writes its partial to the scratch
// (device-coherent stores), waits for them to complete, then counts its arrival; the last of the
// tile's splits (which resets the counter) invalidates its caches and sums all partials in split
// order, so the result does not depend on arrival order.
template <int NPASS, int EPI, bool XG = false>
__device__ __forceinline__ void finish(const GemmParams& p, float (&v)[NPASS][8], int tile_id,
                                       int z, int row0, int grp, int rows_in_tile,
                                       uint32_t* s_last, const EpiCol& ec,
                                       const EpiRow (&er)[NPASS]) {
    const int tid = threadIdx.x;
    if (p.splits > 1) {
        // [tile][split][pass][half][thread] float4s: coalesced stores and loads.
        float* part = p.ws + (size_t)(tile_id * p.splits) * NPASS * 2 * 256 * 4;
        float* mine = part + (size_t)z * NPASS * 2 * 256 * 4;
#pragma unroll
        for (int ps = 0; ps < NPASS; ps++)
#pragma unroll
            for (int h = 0; h < 2; h++)
                xstore16(mine + ((ps * 2 + h) * 256 + tid) * 4,
                         make_float4(v[ps][4 * h], v[ps][4 * h + 1], v[ps][4 * h + 2], v[ps][4 * h + 3]));
        release_wait();
        __syncthreads();
        if (tid == 0) {
            const uint32_t old = atomic_add_agent(p.counters + tile_id, 1u);
            const uint32_t last = old == (uint32_t)(p.splits - 1);
            if (last) atomic_store_agent(p.counters + tile_id, 0u);
            *s_last = last;
        }
        __syncthreads();
        const uint32_t last = *s_last;
        __syncthreads();  // every thread has read s_last before anyone can write it again
        if (last == 0) return;
#pragma unroll
        for (int ps = 0; ps < NPASS; ps++)
#pragma unroll
            for (int e = 0; e < 8; e++) v[ps][e] = 0.0f;
        for (int zz = 0; zz < p.splits; zz++) {
            const float* src = part + (size_t)zz * NPASS * 2 * 256 * 4;
#pragma unroll
            for (int ps = 0; ps < NPASS; ps++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const float4 q = xload16f(src + ((ps * 2 + h) * 256 + tid) * 4);
                    v[ps][4 * h] += q.x;
                    v[ps][4 * h + 1] += q.y;
                    v[ps][4 * h + 2] += q.z;
                    v[ps][4 * h + 3] += q.w;
                }
        }
    }
    const int c0 = (tid & 7) * 4;
#pragma unroll
    for (int ps = 0; ps < NPASS; ps++) {
        const int r = ps * 32 + (tid >> 3);
        const int row = row0 + r;
        epi_apply<EPI, XG>(p, row, grp, c0, v[ps], r < rows_in_tile && row < p.m, ec, er[ps]);
    }
}

// Task `task` (of tiles_n * tiles_m * splits; XCD-mapped) of c = epilogue(a . w^T). The four
// waves split the tile's K steps between them; `red` is lat_lds_floats<BM>() floats of LDS.
// Every thread of the block calls it; it ends with a block barrier, so the caller may reuse
// `red` right after.
template <int BM, int EPI, bool XG = false>
__device__ __forceinline__ void gemm_lat_tile(const GemmParams& p, int task, float* red,
                                              uint32_t* s_last) {
    constexpr int MI = BM / 16;
    constexpr int NPASS = (BM + 31) / 32;
    const int T = p.tiles_n * p.tiles_m * p.splits;
    const int L = xcd_task(task, T);
    const int z = L % p.splits, t2 = L / p.splits;
    const int by = t2 % p.tiles_m, bx = t2 / p.tiles_m;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r16 = l & 15, g = l >> 4;

    // This block's K steps (32 wide), then this wave's quarter of them.
    const int U = p.k >> 5;
    const int ub = z * U / p.splits, ue = (z + 1) * U / p.splits, nu = ue - ub;
    const int u0 = ub + w * nu / 4, u1 = ub + (w + 1) * nu / 4;

    const f16* ap[MI];
    const f16* wp[4];
#pragma unroll
    for (int i = 0; i < MI; i++) {
        const int row = min(by * BM + 16 * i + r16, p.m - 1);  // rows past m: read, never stored
        ap[i] = (const f16*)p.a + (size_t)row * p.k + 8 * g;
    }
    // w in fragment order: unit uu's fragment j is 512 values at ((bx U + uu) 4 + j) 512, and
    // lane l's 8 of them at l * 8 (W rows bx 64 + 16 j + l % 16, K 32 uu + 8 (l / 16) + e).
#pragma unroll
    for (int j = 0; j < 4; j++) wp[j] = (const f16*)p.w + ((size_t)bx * U * 4 + j) * 512 + l * 8;

    // The epilogue's other inputs, in flight with the first operand loads.
    const int c0 = (tid & 7) * 4;
    EpiCol ec;
    EpiRow er[NPASS];
    epi_load_col<EPI>(p, bx, c0, ec);
#pragma unroll
    for (int ps = 0; ps < NPASS; ps++) epi_load_row<EPI, XG>(p, by * BM + ps * 32 + (tid >> 3), bx, c0, er[ps]);

    floatx4 acc[MI][4];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    // The wave's K steps in chunks of up to UMAX, each chunk's fragments all loaded before its
    // MFMAs: a small tile's K loop is latency-bound, so one round trip per chunk instead of one
    // per step. The a operand (an activation) comes through the coherent path when XG.
    //
    // The loads are unconditional (a step past the wave's range re-reads its last step, and its
    // a fragment is masked to zero without a branch): a guarded load becomes a branch, and the
    // compiler drains every outstanding load at each branch, which would serialise the steps.
    constexpr int UMAX = MI == 1 ? 9 : (MI == 2 ? 6 : 4);
    for (int u = u0; u < u1; u += UMAX) {
        half8 fa[UMAX][MI], fw[UMAX][4];
#pragma unroll
        for (int s = 0; s < UMAX; s++) {
            const int uu = min(u + s, u1 - 1);
#pragma unroll
            for (int j = 0; j < 4; j++) fw[s][j] = *(const half8*)(wp[j] + (size_t)uu * 2048);
#pragma unroll
            for (int i = 0; i < MI; i++) fa[s][i] = load16h<XG>(ap[i] + uu * 32);
        }
        // Keep the scheduler from interleaving the MFMAs into the loads (it would reuse the
        // fragment registers and wait for each step's loads before issuing the next).
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < UMAX; s++) {
            const uint32_t keep = u + s < u1 ? 0xffffffffu : 0u;
#pragma unroll
            for (int i = 0; i < MI; i++) {
                const half8 a = mask16(fa[s][i], keep);
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = mfma16(fw[s][j], a, acc[i][j]);
            }
        }
    }

    // acc[i][j] lane: row 16 i + r16, columns 16 j + 4 g + e of the tile. Wave w's partial at
    // red[w][row][col] (rows of 68 floats).
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            *(floatx4*)&red[(w * BM + 16 * i + r16) * 68 + 16 * j + 4 * g] = acc[i][j];
    __syncthreads();

    float v[NPASS][8];
#pragma unroll
    for (int ps = 0; ps < NPASS; ps++) {
        const int r = ps * 32 + (tid >> 3);
#pragma unroll
        for (int e = 0; e < 8; e++) v[ps][e] = 0.0f;
        if (r < BM) {
#pragma unroll
            for (int ww = 0; ww < 4; ww++) {
                const float4 lo = *(const float4*)&red[(ww * BM + r) * 68 + c0];
                const float4 hi = *(const float4*)&red[(ww * BM + r) * 68 + 32 + c0];
                v[ps][0] += lo.x, v[ps][1] += lo.y, v[ps][2] += lo.z, v[ps][3] += lo.w;
                v[ps][4] += hi.x, v[ps][5] += hi.y, v[ps][6] += hi.z, v[ps][7] += hi.w;
            }
        }
    }
    __syncthreads();  // red is free again
    finish<NPASS, EPI, XG>(p, v, bx * p.tiles_m + by, z, by * BM, bx, BM, s_last, ec, er);
}

}  // namespace jh
