// One output tile of the throughput GEMM (BM = 128 or 256 rows x 128 columns), as a device
// function: the body of the per-GEMM `gemm_big` kernel for large M, and a task of the persistent
// encoder kernel on large batches. c = epilogue(a . w^T) as the latency tile computes it.
//
// The K loop runs BK = 64 at a time through three LDS stages filled by direct global -> LDS
// loads (no register staging), so the copies of stages k + 1 and k + 2 are in flight while stage
// k feeds the MFMAs, with one block barrier per stage.
//  - a's stage: BM rows x 128 bytes; wave load I takes rows 8 I .. 8 I + 7 whole (8 lanes a row:
//    full 128-byte lines from memory), lane l into LDS chunk 64 I + l, which is row r = 8 I + l / 8,
//    chunk l % 8, and holds a's chunk (l % 8) ^ ((r / 2) % 8) of that row: the 16 rows a fragment
//    read touches (two per bank half) land on 16 different banks.
//  - w's stage: two 64-row groups x two 32-wide K units of the fragment-ordered matrix, copied
//    as they are (16 KB, contiguous per group).
// Four waves in a 2 x 2 grid each own (BM / 2) x 64 outputs with MFMA 32 x 32 x 16 (a single wave
// per SIMD issues it at ~82% of the f16 peak, 16 x 16 x 32 at ~52%): MR = BM / 64 row fragments x
// 2 column fragments, w as the A operand (a lane gets 4 groups of 4 consecutive output columns of
// one row). A 32-row, 16-wide K slice of the fragment order is four 16-byte chunks a lane can
// address directly, so the packed weights serve this MFMA shape too. The finished tile goes
// through LDS, one 64-column group at a time, into finish() / the epilogue.
#pragma once

#include "gemm_tile.h"

namespace jh {

template <int BM>
struct Big {
    static constexpr int BN = 128, BK = 64;
    static constexpr int WM = BM / 2, MR = WM / 32;        // wave rows, 32-row fragments per wave
    static constexpr int A_BYTES = BM * BK * 2, W_BYTES = BN * BK * 2;
    static constexpr int STAGE = A_BYTES + W_BYTES;         // bytes per stage
    static constexpr int LOADS = STAGE / 1024 / 4;          // 1 KB wave loads per wave per stage
    static constexpr int OUT_BYTES = BM * 68 * 4;           // one 64-column group of f32 outputs
    static constexpr int LDS_BYTES = 3 * STAGE > OUT_BYTES ? 3 * STAGE : OUT_BYTES;
};

// s_waitcnt with vmcnt = n (n < 16) and no wait on the other counters (gfx9 encoding:
// vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 16, "vmcnt field");
    __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// Task `task` of tiles_n * tiles_m * splits (XCD-mapped; consecutive tasks of an XCD share a's
// rows and walk w's column groups, so an XCD reads its a rows once and w stays in its L2).
// AX: a is read device-coherent; XG: the outputs are stored and the statistics read
// device-coherent. The residual is read through the caches (c itself in a per-GEMM launch, or
// the persistent kernel's write-once p.res).
template <int BM, int EPI, bool AX, bool XG>
__device__ __forceinline__ void gemm_big_tile(const GemmParams& p, int task, char* lds,
                                              uint32_t* s_last) {
    using C = Big<BM>;
    constexpr int NPASS = BM / 32;
    const int T = p.tiles_n * p.tiles_m * p.splits;
    const int L = xcd_task(task, T);
    const int z = L % p.splits, t2 = L / p.splits;
    const int bx = t2 % p.tiles_n, by = t2 / p.tiles_n;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int wm = w >> 1, wn = w & 1;
    const int U = p.k >> 5, KT = p.k >> 6;
    const int kt0 = z * KT / p.splits, kt1 = (z + 1) * KT / p.splits, nkt = kt1 - kt0;

    // The epilogue's other inputs for both 64-column groups, in flight with the first stages.
    const int c0 = (tid & 7) * 4;
    EpiCol ec[2];
    EpiRow er[2][NPASS];
#pragma unroll
    for (int gg = 0; gg < 2; gg++) {
        epi_load_col<EPI>(p, bx * 2 + gg, c0, ec[gg]);
#pragma unroll
        for (int ps = 0; ps < NPASS; ps++)
            epi_load_row<EPI, XG, false>(p, by * BM + ps * 32 + (tid >> 3), bx * 2 + gg, c0, er[gg][ps]);
    }
#pragma unroll
    for (int gg = 0; gg < 2; gg++)
#pragma unroll
        for (int ps = 0; ps < NPASS; ps++) epi_load_rope<EPI>(p, c0, er[gg][ps]);

    // Stage copies: wave w issues loads I = w, w + 4, ... of the stage's A_BYTES / 1024 a loads
    // then W_BYTES / 1024 w loads.
    auto issue = [&](int kt, int buf) {
        char* st = lds + buf * C::STAGE;
#pragma unroll
        for (int q = 0; q < C::LOADS; q++) {
            const int I = w + 4 * q;
            if (I < C::A_BYTES / 1024) {
                const int r = 8 * I + (l >> 3), ch = (l & 7) ^ ((r >> 1) & 7);
                const int row = min(by * BM + r, p.m - 1);
                const f16* src = (const f16*)p.a + (size_t)row * p.k + kt * 64 + ch * 8;
                lds_dma16<AX>(src, st + I * 1024);
            } else {
                const int J = I - C::A_BYTES / 1024;  // 4 KB block J / 4 = (group, unit), part J % 4
                const int blk = J >> 2, G = bx * 2 + (blk >> 1), u = 2 * kt + (blk & 1);
                const f16* src = (const f16*)p.w + ((size_t)(G * U + u) * 4 + (J & 3)) * 512 + l * 8;
                lds_dma16<false>(src, st + C::A_BYTES + J * 1024);
            }
        }
    };

    floatx16 acc[C::MR][2];
#pragma unroll
    for (int i = 0; i < C::MR; i++)
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][c][e] = 0.0f;

    if (nkt > 0) issue(kt0, 0);
    if (nkt > 1) issue(kt0 + 1, 1);
    const int l32 = l & 31, hi = l >> 5;
    for (int s = 0; s < nkt; s++) {
        // This wave's copies of stage s are done (the next stage's may stay in flight), then a
        // bare barrier: every wave's are, and every wave is done reading stage s - 1, whose
        // buffer the copy issued next overwrites. (__syncthreads' release fence would wait for
        // all of this wave's copies, the next stage's too.)
        if (s + 1 < nkt)
            wait_vmcnt<C::LOADS>();
        else
            wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        if (s + 2 < nkt) issue(kt0 + s + 2, (s + 2) % 3);
        const char* st = lds + (s % 3) * C::STAGE;
        const char* ws = st + C::A_BYTES;
        // Four K-16 steps t. Lane l takes K 16 t + 8 (l / 32) .. + 7: a's chunk 2 t + l / 32 of row
        // 32 i + l % 32; w's row 32 c + l % 32 of the wave's 64-column group, which in the
        // fragment order is unit t / 2, fragment 2 c + (l % 32) / 16, lane group 2 (t % 2) + l / 32.
        // Step t + 1's fragments are read while step t's MFMAs run (two register sets).
        half8 fa[2][C::MR], fw[2][2];
        auto rd = [&](int t) {
            const int b = t & 1;
#pragma unroll
            for (int i = 0; i < C::MR; i++) {
                const int r = wm * C::WM + 32 * i + l32;
                fa[b][i] = *(const half8*)(st + (r * 8 + ((2 * t + hi) ^ ((r >> 1) & 7))) * 16);
            }
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const int j = 2 * c + (l32 >> 4), g2 = 2 * (t & 1) + hi;
                fw[b][c] = *(const half8*)(ws + ((wn * 2 + (t >> 1)) * 4 + j) * 1024 + (g2 * 16 + (l & 15)) * 16);
            }
        };
        auto mm = [&](int t) {
            const int b = t & 1;
#pragma unroll
            for (int i = 0; i < C::MR; i++)
#pragma unroll
                for (int c = 0; c < 2; c++)
                    acc[i][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fw[b][c], fa[b][i], acc[i][c], 0, 0, 0);
        };
        rd(0);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            if (t + 1 < 4) rd(t + 1);
            __builtin_amdgcn_sched_barrier(0);  // the next step's reads ahead of this step's MFMAs
            mm(t);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __syncthreads();  // every wave is done with the stages: the outputs reuse the space

    // The output through LDS (f32, rows of 64 + 4 pad), one 64-column group (the waves with
    // wn == grp) at a time, into the epilogue layout.
    float* out = (float*)lds;
#pragma unroll
    for (int grp = 0; grp < 2; grp++) {
        if (wn == grp) {  // acc[i][c][4 q + e]: row 32 i + l % 32, column 32 c + 8 q + 4 (l / 32) + e
#pragma unroll
            for (int i = 0; i < C::MR; i++)
#pragma unroll
                for (int c = 0; c < 2; c++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        *(floatx4*)&out[(wm * C::WM + 32 * i + l32) * 68 + 32 * c + 8 * q + 4 * hi] =
                            floatx4{acc[i][c][4 * q], acc[i][c][4 * q + 1], acc[i][c][4 * q + 2],
                                    acc[i][c][4 * q + 3]};
        }
        __syncthreads();
        float v[NPASS][8];
#pragma unroll
        for (int ps = 0; ps < NPASS; ps++) {
            const float* src = &out[(ps * 32 + (tid >> 3)) * 68 + c0];
            const float4 lo = *(const float4*)src, hi = *(const float4*)(src + 32);
            v[ps][0] = lo.x, v[ps][1] = lo.y, v[ps][2] = lo.z, v[ps][3] = lo.w;
            v[ps][4] = hi.x, v[ps][5] = hi.y, v[ps][6] = hi.z, v[ps][7] = hi.w;
        }
        __syncthreads();  // every thread has read the group before the next one is written
        // Each 64-column group is its own split-K "tile" (two per block).
        finish<NPASS, EPI, XG>(p, v, (bx * p.tiles_m + by) * 2 + grp, z, by * BM, bx * 2 + grp, BM,
                               s_last, ec[grp], er[grp]);
    }
}

}  // namespace jh
