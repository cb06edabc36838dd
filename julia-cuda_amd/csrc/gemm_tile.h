// One output tile of the latency GEMM (BM = 16/32/48/64 rows x 64 columns), as a device function:
// the body of the per-GEMM `gemm_lat` kernels and a task of the persistent layer kernel, which
// pass their own LDS. See gemm.hip for the design.
#pragma once

#include <type_traits>

#include "device.h"

namespace jh {

// The LDS slot (floats) of one wave of a BM-row latency tile: its partial BM x 64 tile (rows
// padded to 68 floats); with eight waves also its staged activation lines first (lat_stage_lines
// lines of 128 bytes a row: 32 floats each), as many of four, three or two as fit the CU's 160 KB.
template <int BM, int NW>
constexpr int lat_stage_lines() {
    return NW != 8 ? 0 : 8 * BM * 128 * 4 <= 150 * 1024 ? 4 : 8 * BM * 96 * 4 <= 150 * 1024 ? 3 : 2;
}
template <int BM, int NW>
constexpr int lat_slot_floats() {
    return BM * 68 > BM * 32 * lat_stage_lines<BM, NW>() ? BM * 68 : BM * 32 * lat_stage_lines<BM, NW>();
}
// LDS floats gemm_lat_tile<BM> needs with NW waves.
template <int BM, int NW = 4>
constexpr int lat_lds_floats() { return NW * lat_slot_floats<BM, NW>(); }

// The K path of an eight-wave latency tile's waves, when the kernel fixes it: every wave in one
// chunk of three, five or six K steps (LAT_KONE3, LAT_KONE5, LAT_KONE6: tiles of up to 32 rows,
// whose six steps' four lines of a a row fit the LDS) or in the chunked loop (LAT_KLOOP);
// LAT_KANY chooses per wave at run time. One path per kernel keeps the waits exact: the compiler
// joins run-time alternatives into one flow, and each alternative then waits for the loads the
// others might have left in flight (measured in the generated code: a full wait ahead of the
// three-step chunk's weight loads, for the other paths' RoPE table loads).
enum { LAT_KANY = 0, LAT_KLOOP = 1, LAT_KONE3 = 3, LAT_KONE5 = 5, LAT_KONE6 = 6 };

// Rows of one epilogue pass of a four-wave latency tile (256 threads, 8 a row): the unit in which
// a K split's partial tile is stored (gemm_ws_floats sizes the scratch by it). Only four-wave
// tiles take a K split.
constexpr int LAT_SPLIT_PASS_ROWS = 32;

// Shared tail: each thread's 8 values (K fully summed within the block) -> the split-K
// reduction when the grid splits K -> the epilogue. Thread t of NT owns row (pass * NT / 8 +
// t / 8) of the tile and columns c0 = 4 (t % 8), c0 + 32 of 64-column group `grp`.
//
// Split-K (kernels/src/gemm.rs:355-433): every block writes its partial to the scratch
// (device-coherent stores), waits for them to complete, then counts its arrival; the last of the
// tile's splits (which resets the counter) invalidates its caches and sums all partials in split
// order, so the result does not depend on arrival order.
template <int NPASS, int EPI, bool XG = false, int NT = 256>
__device__ __forceinline__ void finish(const GemmParams& p, float (&v)[NPASS][8], int tile_id,
                                       int z, int row0, int grp, int rows_in_tile,
                                       uint32_t* s_last, const EpiCol& ec,
                                       const EpiRow (&er)[NPASS]) {
    const int tid = threadIdx.x;
    if (p.splits > 1) {
        // [tile][split][pass][half][thread] float4s: coalesced stores and loads.
        // (one buffer descriptor over the tile's partials: 16-byte coherent stores and loads)
        const auto part = buffer_rsrc(p.ws + (size_t)(tile_id * p.splits) * NPASS * 2 * NT * 4,
                                      p.splits * NPASS * 2 * NT * 16);
        const uint32_t mine = (uint32_t)z * NPASS * 2 * NT * 16;
#pragma unroll
        for (int ps = 0; ps < NPASS; ps++)
#pragma unroll
            for (int h = 0; h < 2; h++)
                bstore16f(part, mine + ((ps * 2 + h) * NT + tid) * 16,
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
            const uint32_t src = (uint32_t)zz * NPASS * 2 * NT * 16;
#pragma unroll
            for (int ps = 0; ps < NPASS; ps++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const float4 q = bload16f(part, src + ((ps * 2 + h) * NT + tid) * 16);
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
        const int r = ps * (NT / 8) + (tid >> 3);
        const int row = row0 + r;
        epi_apply<EPI, XG>(p, row, grp, c0, v[ps], r < rows_in_tile && row < p.m, ec, er[ps]);
    }
    if (EPI & EPI_SCORE) {
        // Every tile's partials are stored (device-coherent) before its arrival counts; the last
        // tile to arrive (which resets the counter) sums each row's partials in column order.
        release_wait();
        __syncthreads();
        if (tid == 0) {
            const uint32_t old = atomic_add_agent(p.counters, 1u);
            const uint32_t last = old == (uint32_t)(p.tiles_n * p.tiles_m - 1);
            if (last) atomic_store_agent(p.counters, 0u);
            *s_last = last;
        }
        __syncthreads();
        const uint32_t last = *s_last;
        __syncthreads();  // every thread has read s_last before anyone can write it again
        if (last) {
            for (int r = tid; r < p.m; r += NT) {
                float acc = 0.0f;
                for (int t = 0; t < p.tiles_n; t++) acc += xload32(p.ws + (size_t)r * p.tiles_n + t);
                p.logits[r] = acc + p.score_b;
            }
        }
    }
}

// Task `task` (of tiles_n * tiles_m * splits; XCD-mapped) of c = epilogue(a . w^T). The NW
// waves split the tile's K steps between them; `red` is lat_lds_floats<BM, NW>() floats of LDS.
// Every thread of the block calls it; it ends with a block barrier, so the caller may reuse
// `red` right after. ONE: the block has its CU to itself (four waves: 512 registers a lane),
// so that the 48- and 64-row tiles hold every K step of a wave in flight at once. Eight waves
// (NW = 8) take a CU's operand loads at a higher rate than four.
template <int BM, int EPI, bool XG = false, bool ONE = false, int NW = 4, int KP = LAT_KANY>
__device__ __forceinline__ void gemm_lat_tile(const GemmParams& p, int task, float* red,
                                              uint32_t* s_last, uint64_t* sub = nullptr) {
    auto mark = [&](int i) {  // profiling: thread 0's view of the task's stages
        if (sub && threadIdx.x == 0) sub[i] = wall_clock64();
    };
    mark(0);
    constexpr int MI = BM / 16;
    constexpr int RPP = 8 * NW;                     // tile rows a pass of the epilogue
    constexpr int NPASS = (BM + RPP - 1) / RPP;
    constexpr int SLOT = lat_slot_floats<BM, NW>();  // a wave's LDS floats
    static_assert(NW != 4 || RPP == LAT_SPLIT_PASS_ROWS, "split partials are sized by 32-row passes");
    const int T = p.tiles_n * p.tiles_m * p.splits;
    const int L = xcd_task(task, T);
    const int z = L % p.splits, t2 = L / p.splits;
    const int by = t2 % p.tiles_m, bx = t2 / p.tiles_m;
    const int tid = threadIdx.x, l = tid & 63, r16 = l & 15, g = l >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches

    // This block's K steps (32 wide), then this wave's share of them.
    const int U = p.k >> 5;
    const int ub = z * U / p.splits, ue = (z + 1) * U / p.splits, nu = ue - ub;
    const int u0 = ub + w * nu / NW, u1 = ub + (w + 1) * nu / NW;
    // Eight waves, each with its K steps in one chunk (up to 40 steps a split; 48 on the six-step
    // path): the waves'
    // partials are summed in two halves. The operands reach the CU in the order the waves issued
    // their loads, so waves 4-7 (each the second wave of its SIMD) finish ~1.5 us after waves
    // 0-3 (293 rows, K = 768), and waves 0-3 sum their four partials in that time; after the
    // last wave only the half sum and four partials remain. The late waves pass the first barrier
    // right after issuing their loads. The sums run in wave order either way (the values do not
    // depend on which half finishes first).
    // (block-uniform: every wave takes kone)
    const bool two = NW == 8 && (KP == LAT_KONE6 || (nu + NW - 1) / NW <= 5);
    const bool late = two && w >= NW / 2;

    const f16* ap[MI];
#pragma unroll
    for (int i = 0; i < MI; i++) {
        const int row = min(by * BM + 16 * i + r16, p.m - 1);  // rows past m: read, never stored
        ap[i] = (const f16*)p.a + (size_t)src_row<EPI>(p, row) * p.k + 8 * g;
    }
    // Eight waves with K ranges of up to three or five units: a goes through the wave's LDS slot
    // as whole 128-byte lines (see kone), copied first, before any other load of the tile. The
    // copies go through a buffer descriptor over a (the host checks that it spans at most 4 GB):
    // the compiler counts buffer copies in order with the other loads, so the waits that follow
    // are partial. (With global-address copies in flight it waits for every load instead.)
    constexpr int NLS = lat_stage_lines<BM, NW>();
    static_assert(NLS == 0 || NLS * BM * 32 <= SLOT, "the staged lines fit the wave's slot");
    char* const slot = (char*)(red + w * SLOT);
    const int L0 = u0 >> 1;  // the first line of the wave's K range
    auto swz = [](int r) { return (r & 7) ^ ((r >> 3) & 1); };
    // Lane l copies 16 bytes of row 8 rb + l / 8 a copy: one lane offset a row block (aoff,
    // kept live until the fragment loads have gone out: the compiler would otherwise give their
    // registers to w's fragments and wait for the copies first), the line as a scalar offset.
    uint32_t aoff[NLS ? BM / 8 : 1];
    auto stage_a = [&](auto nl_) {
        constexpr int NL = decltype(nl_)::value;  // lines a row the wave's K range touches
        const int a_rows = (EPI & EPI_GATHER) ? p.src_m : p.m;
        const auto ar = buffer_rsrc(p.a, (uint32_t)((size_t)a_rows * p.k * 2));
#pragma unroll
        for (int rb = 0; rb < BM / 8; rb++) {
            const int r = 8 * rb + (l >> 3);
            const int row = min(by * BM + r, p.m - 1);  // rows past m: read, never stored
            aoff[rb] = ((uint32_t)src_row<EPI>(p, row) * (uint32_t)p.k +
                        (uint32_t)(L0 * 64 + ((l & 7) ^ swz(r)) * 8)) * 2u;
        }
#pragma unroll
        for (int li = 0; li < NL; li++) {
            const uint32_t soff = (uint32_t)(min(L0 + li, (p.k >> 6) - 1) - L0) * 128u;  // wave-uniform
#pragma unroll
            for (int rb = 0; rb < BM / 8; rb++)
                lds_bdma16<XG>(ar, aoff[rb], slot + (li * (BM / 8) + rb) * 1024, soff);
        }
    };
    static_assert(KP == LAT_KANY || NW == 8, "a fixed K path is an eight-wave tile's");
    if constexpr (KP == LAT_KONE3) {
        stage_a(std::integral_constant<int, 2>{});
    } else if constexpr (KP == LAT_KONE5) {
        if constexpr (NLS >= 3) stage_a(std::integral_constant<int, 3>{});
    } else if constexpr (KP == LAT_KONE6) {
        static_assert(NLS >= 4, "six K steps' lines staged");
        stage_a(std::integral_constant<int, 4>{});
    } else if constexpr (KP == LAT_KANY) {
        const int nuw = u1 - u0;
        if (NW == 8 && nuw <= 3 && NLS >= 2) stage_a(std::integral_constant<int, 2>{});
        else if (NW == 8 && nuw > 3 && nuw <= 5 && NLS >= 3) stage_a(std::integral_constant<int, 3>{});
    }

    // The epilogue's other inputs, in flight with the first operand loads.
    const int c0 = (tid & 7) * 4;
    EpiCol ec;
    EpiRow er[NPASS];
    epi_load_col<EPI>(p, bx, c0, ec);
#pragma unroll
    for (int ps = 0; ps < NPASS; ps++) epi_load_row<EPI, XG>(p, by * BM + ps * RPP + (tid >> 3), bx, c0, er[ps]);

    floatx4 acc[MI][4];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    // The wave's K steps in chunks of UC, two chunks in flight: chunk c + 1's fragments load
    // while chunk c's MFMAs run, so a wave pays one round trip to memory however many chunks its
    // K range takes. The a operand (an activation) comes through the coherent path when XG.
    //
    // The loads are unconditional within a chunk (a step past the wave's range re-reads its last
    // step, and its a fragment is masked to zero without a branch): a guarded load becomes a
    // branch, and the compiler drains every outstanding load at each divergent branch, which would
    // serialise the steps. The chunk guards depend on the wave index only (scalar branches).
    // UC K steps a chunk (2 x UC x (MI + 4) x 4 VGPRs of fragments): four, three or two; five for
    // 16-row tiles whose waves have more than eight K steps (K = 1152), which then take one round
    // trip instead of two. With a CU to itself (ONE), three or five for 32-row tiles and up: one
    // round trip up to 10 K steps a wave.
    auto kloop = [&](auto uc_) {
        constexpr int UC = decltype(uc_)::value;
        half8 fa0[UC][MI], fw0[UC][4], fa1[UC][MI], fw1[UC][4];
        // w in fragment order: unit uu's fragment j is 512 values at ((bx U + uu) 4 + j) 512,
        // and lane l's 8 of them at l * 8 (W rows bx 64 + 16 j + l % 16, K 32 uu + 8 (l / 16) +
        // e); read through a buffer descriptor over exactly the wave's K steps: a slot past them
        // reads zeros without touching memory (a clamped re-read would still cost its bytes).
        const auto wr = buffer_rsrc((const f16*)p.w + ((size_t)bx * U + u0) * 2048,
                                    (uint32_t)(u1 - u0) * 4096);
        auto load = [&](half8 (&fa)[UC][MI], half8 (&fw)[UC][4], int u) {
#pragma unroll
            for (int s = 0; s < UC; s++) {
                const int uu = min(u + s, u1 - 1);
#pragma unroll
                for (int j = 0; j < 4; j++)
                    fw[s][j] = bload16<false>(wr, (uint32_t)(u + s - u0) * 4096 + j * 1024 + l * 16);
#pragma unroll
                for (int i = 0; i < MI; i++) fa[s][i] = load16h<XG>(ap[i] + uu * 32);
            }
        };
        auto compute = [&](const half8 (&fa)[UC][MI], const half8 (&fw)[UC][4], int u) {
#pragma unroll
            for (int s = 0; s < UC; s++) {
                const uint32_t keep = u + s < u1 ? 0xffffffffu : 0u;
#pragma unroll
                for (int i = 0; i < MI; i++) {
                    const half8 a = mask16(fa[s][i], keep);
#pragma unroll
                    for (int j = 0; j < 4; j++) acc[i][j] = mfma16(fw[s][j], a, acc[i][j]);
                }
            }
        };
        // (Scheduling fences keep the compiler from interleaving the MFMAs into the loads, where
        // it would reuse the fragment registers and wait for each step's loads before the next.)
        // The first two chunks unconditionally (every wave has a K step: the host checks; a slot
        // past the wave's range re-reads its last a step and reads zeros of w), so that the
        // compiler knows where the position loads stand in the load order when the table loads
        // wait for them.
        load(fa0, fw0, u0);
        load(fa1, fw1, u0 + UC);
        // The RoPE table rows after the operand loads: they wait for the positions, and issued
        // first that wait would hold back the operand loads by a round trip.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ps = 0; ps < NPASS; ps++) epi_load_rope<EPI>(p, by * BM + ps * RPP + (tid >> 3), c0, er[ps]);
        for (int u = u0; u < u1; u += 2 * UC) {
            __builtin_amdgcn_sched_barrier(0);
            compute(fa0, fw0, u);
            __builtin_amdgcn_sched_barrier(0);
            if (u + 2 * UC < u1) load(fa0, fw0, u + 2 * UC);
            __builtin_amdgcn_sched_barrier(0);
            if (u + UC < u1) compute(fa1, fw1, u + UC);
            __builtin_amdgcn_sched_barrier(0);
            if (u + 3 * UC < u1) load(fa1, fw1, u + 3 * UC);
        }
    };
    // Every K step of the wave in one chunk (eight waves: three to five steps a wave).
    //
    // With LDS staging (STAGE: the wave's K range spans at most NL 128-byte lines a row, and its
    // slot holds them), a is copied into the wave's own LDS slot as whole lines and the fragments
    // are read from there. A fragment load straight from memory takes 16 rows x 64 bytes (the
    // MFMA gives lane l row l % 16 and 8 K values of a 32-wide unit), half a 128-byte line a
    // row, so the next unit's load asks for the same lines again; a CU's intake follows the
    // number of line requests more than the bytes (measured at 293 rows: time ~ 2.2 us + 2 ns a
    // line request over the tile heights, the same for 16 x 64 and 32 x 32 tiles of equal
    // request counts). A direct copy here takes 8 rows x 128 bytes: half the requests for a.
    // Copy q = line x (BM / 8) + rb holds rows 8 rb .. 8 rb + 7 of line L0 + line at slot bytes
    // 1024 q + 128 (r % 8) + 16 (c ^ sw(r)), c the 16-byte chunk of the line, sw(r) = (r % 8) ^
    // ((r / 8) % 2): the 16 rows one fragment read takes cover the 64 banks.
    auto kone = [&](auto uc_, auto stage_) {
        constexpr int UC = decltype(uc_)::value;
        constexpr bool STAGE = decltype(stage_)::value;
        half8 fa[UC][MI], fw[UC][4];
        const auto wr = buffer_rsrc((const f16*)p.w + ((size_t)bx * U + u0) * 2048,
                                    (uint32_t)(u1 - u0) * 4096);
#pragma unroll
        for (int s = 0; s < UC; s++) {
            const int uu = min(u0 + s, u1 - 1);
#pragma unroll
            for (int j = 0; j < 4; j++) fw[s][j] = bload16<false>(wr, (uint32_t)s * 4096 + j * 1024 + l * 16);
            if (!STAGE) {
#pragma unroll
                for (int i = 0; i < MI; i++) fa[s][i] = load16h<XG>(ap[i] + uu * 32);
            }
        }
        if (STAGE) {
#pragma unroll
            for (int rb = 0; rb < BM / 8; rb++) asm volatile("" ::"v"(aoff[rb]));
        }
        __builtin_amdgcn_sched_barrier(0);
        // The RoPE table loads wait for the positions. While copies into LDS are in flight the
        // compiler takes any such wait as one for every load (it does not count the copies in
        // order with the other loads), so with STAGE they follow the explicit wait below.
        if (!STAGE) {
#pragma unroll
            for (int ps = 0; ps < NPASS; ps++) epi_load_rope<EPI>(p, by * BM + ps * RPP + (tid >> 3), c0, er[ps]);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (late) __builtin_amdgcn_s_barrier();  // the halves' first barrier (see `two`)
        __builtin_amdgcn_sched_barrier(0);
        if (STAGE) {
            // The copies went out before every other load of the tile (stage_a): waiting until
            // at most w's 4 UC fragment loads are in flight covers them.
            wait_vmcnt<4 * UC>();
#pragma unroll
            for (int ps = 0; ps < NPASS; ps++) epi_load_rope<EPI>(p, by * BM + ps * RPP + (tid >> 3), c0, er[ps]);
#pragma unroll
            for (int s = 0; s < UC; s++) {
                const int uu = min(u0 + s, u1 - 1);
#pragma unroll
                for (int i = 0; i < MI; i++) {
                    const int r = 16 * i + r16, c = 4 * (uu & 1) + g;
                    const int q = ((uu >> 1) - L0) * (BM / 8) + (r >> 3);
                    fa[s][i] = *(const half8*)(slot + q * 1024 + (r & 7) * 128 + 16 * (c ^ swz(r)));
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < UC; s++) {
            const uint32_t keep = u0 + s < u1 ? 0xffffffffu : 0u;
#pragma unroll
            for (int i = 0; i < MI; i++) {
                const half8 a = mask16(fa[s][i], keep);
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = mfma16(fw[s][j], a, acc[i][j]);
            }
        }
    };
    using ST2 = std::integral_constant<bool, (lat_stage_lines<BM, NW>() >= 2)>;
    using ST3 = std::integral_constant<bool, (lat_stage_lines<BM, NW>() >= 3)>;
    if constexpr (KP == LAT_KONE3) {
        kone(std::integral_constant<int, 3>{}, ST2{});
    } else if constexpr (KP == LAT_KONE5) {
        kone(std::integral_constant<int, 5>{}, ST3{});
    } else if constexpr (KP == LAT_KONE6) {
        kone(std::integral_constant<int, 6>{}, std::true_type{});
    } else if (KP == LAT_KANY && NW == 8 && u1 - u0 <= 3) {
        kone(std::integral_constant<int, 3>{}, ST2{});
    } else if (KP == LAT_KANY && NW == 8 && u1 - u0 <= 5) {
        kone(std::integral_constant<int, 5>{}, ST3{});
    } else if (ONE && MI > 1) {
        if (u1 - u0 > 6)
            kloop(std::integral_constant<int, 5>{});
        else
            kloop(std::integral_constant<int, 3>{});
    } else if (MI == 1 && u1 - u0 > 8) {
        kloop(std::integral_constant<int, 5>{});
    } else {
        kloop(std::integral_constant<int, MI == 1 ? 4 : (MI == 2 ? 3 : 2)>{});
    }

    mark(1);
    // acc[i][j] lane: row 16 i + r16, columns 16 j + 4 g + e of the tile. Wave w's partial at
    // red[w][row][col] (rows of 68 floats).
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            *(floatx4*)&red[w * SLOT + (16 * i + r16) * 68 + 16 * j + 4 * g] = acc[i][j];
    // The partials summed in wave order, from slot `from` on (0: all eight; two: the half sum in
    // slot 0, then waves 4-7).
    auto sum_slots = [&](float (&v)[NPASS][8], int from) {
#pragma unroll
        for (int ps = 0; ps < NPASS; ps++) {
            const int r = ps * RPP + (tid >> 3);
#pragma unroll
            for (int e = 0; e < 8; e++) v[ps][e] = 0.0f;
            if (r < BM) {
#pragma unroll
                for (int ww = 0; ww < NW; ww++) {
                    if (ww > 0 && ww < from) continue;
                    const float4 lo = *(const float4*)&red[ww * SLOT + r * 68 + c0];
                    const float4 hi = *(const float4*)&red[ww * SLOT + r * 68 + 32 + c0];
                    v[ps][0] += lo.x, v[ps][1] += lo.y, v[ps][2] += lo.z, v[ps][3] += lo.w;
                    v[ps][4] += hi.x, v[ps][5] += hi.y, v[ps][6] += hi.z, v[ps][7] += hi.w;
                }
            }
        }
    };
    float v[NPASS][8];
    if (two) {
        if (!late) {
            // The early waves' partials are in (the late waves passed this barrier earlier), and
            // their 256 threads sum them into slot 0: 0 + w0 + w1 + w2 + w3, as the full sum
            // would run.
            wait_lgkm0();
            __builtin_amdgcn_s_barrier();
            for (int x = tid; x < BM * 16; x += 64 * (NW / 2)) {
                float* e0 = &red[(x >> 4) * 68 + 4 * (x & 15)];
                float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                for (int ww = 0; ww < NW / 2; ww++) {
                    const float4 b = *(const float4*)(e0 + ww * SLOT);
                    a.x += b.x, a.y += b.y, a.z += b.z, a.w += b.w;
                }
                *(float4*)e0 = a;
            }
        }
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();  // every partial and the half sum are in
        sum_slots(v, NW / 2);
    } else {
        __syncthreads();
        sum_slots(v, 0);
    }
    __syncthreads();  // red is free again
    mark(2);
    finish<NPASS, EPI, XG, 64 * NW>(p, v, bx * p.tiles_m + by, z, by * BM, bx, BM, s_last, ec, er);
    mark(3);
}

// ---- the persistent kernel's tile: weights staged in LDS --------------------------------------
// The weight tile of a task (64 columns x one split's K units, fragment order) is one contiguous
// run of the packed matrix, nu * 4 KB. The persistent kernel copies it into LDS with direct
// global -> LDS loads, if it can before the barrier that precedes the task's phase (the weights
// do not depend on the previous phase), so that after the barrier only the activation loads
// stand between the block and its MFMAs.

struct WTile {
    int bx, ub, nu;  // 64-column group, first K unit, units
};

__device__ __forceinline__ WTile w_tile_of(const GemmParams& p, int task) {
    const int T = p.tiles_n * p.tiles_m * p.splits;
    const int L = xcd_task(task, T);
    const int z = L % p.splits, bx = (L / p.splits) / p.tiles_m;
    const int U = p.k >> 5;
    const int ub = z * U / p.splits;
    return WTile{bx, ub, (z + 1) * U / p.splits - ub};
}

// LDS bytes of the weight tile for splits of a k-wide GEMM (the largest split).
__host__ __device__ constexpr int w_tile_bytes(int k, int splits) {
    return ((k / 32 + splits - 1) / splits) * 4096;
}

// Waves [w_first, 4) copy task's weight tile to `lds` (1 KB per wave load). (Global copies: the
// same copies through a buffer descriptor made the whole-model launch 13-19% slower, the
// prefetch no longer overlapping what runs before the tile's wait.)
__device__ __forceinline__ void w_tile_fetch(const GemmParams& p, WTile t, f16* lds, int w_first) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (w < w_first) return;
    const f16* src = (const f16*)p.w + (size_t)(t.bx * (p.k >> 5) + t.ub) * 2048 + l * 8;
    for (int c = w - w_first; c < 4 * t.nu; c += 4 - w_first) lds_dma16(src + (size_t)c * 512, lds + c * 512);
}

// LDS floats the cross-wave reduction of a BM-row tile needs (aliases the weight tile).
template <int BM>
constexpr int w_red_floats() { return 4 * BM * 68; }

// Task `task` of c = epilogue(a . w^T) in the persistent kernel. The weight tile is in `lds`
// already (w_ready: its loads were issued earlier by this block, maybe still in flight) or is
// fetched here. a is read with 16-byte buffer loads, rows past m reading zeros: device-coherent
// when AX (a buffer other blocks write more than once per launch, or several blocks write parts
// of one line), else through the caches (a buffer written once per launch, each 128-byte line by
// one block: no L2 can hold a stale copy). The statistics are read device-coherent, the residual
// (a write-once buffer) through the caches; the outputs are stored device-coherent. The four
// waves split the tile's K units; their partial tiles are summed through LDS, in the weight
// tile's space. Every thread calls this; it ends with a block barrier after the last LDS access.
template <int BM, int EPI, bool AX>
__device__ __forceinline__ void gemm_w_tile(const GemmParams& p, int task, char* lds, bool w_ready,
                                            uint32_t* s_last, uint64_t* sub = nullptr) {
    auto mark = [&](int i) {  // profiling: thread 0's view of the task's stages
        if (sub && threadIdx.x == 0) sub[i] = wall_clock64();
    };
    constexpr int MI = BM / 16;
    constexpr int NPASS = (BM + LAT_SPLIT_PASS_ROWS - 1) / LAT_SPLIT_PASS_ROWS;
    constexpr int UMAX = MI >= 3 ? 6 : 9;  // a fragments one wave holds: 72-96 or 36-72 VGPRs
    const int T = p.tiles_n * p.tiles_m * p.splits;
    const int L = xcd_task(task, T);
    const int z = L % p.splits, t2 = L / p.splits;
    const int by = t2 % p.tiles_m, bx = t2 / p.tiles_m;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r16 = l & 15, g = l >> 4;
    const int U = p.k >> 5;
    const int ub = z * U / p.splits, nu = (z + 1) * U / p.splits - ub;
    const int u0 = w * nu / 4, u1 = (w + 1) * nu / 4;  // this wave's units, relative to ub
    f16* wl = (f16*)lds;
    if (!w_ready) w_tile_fetch(p, WTile{bx, ub, nu}, wl, 0);

    const int c0 = (tid & 7) * 4;
    EpiCol ec;
    EpiRow er[NPASS];
    epi_load_col<EPI>(p, bx, c0, ec);
#pragma unroll
    for (int ps = 0; ps < NPASS; ps++) epi_load_row<EPI, true, false>(p, by * BM + ps * 32 + (tid >> 3), bx, c0, er[ps]);
#pragma unroll
    for (int ps = 0; ps < NPASS; ps++) epi_load_rope<EPI>(p, by * BM + ps * 32 + (tid >> 3), c0, er[ps]);

    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(p.a, (uint32_t)p.m * (uint32_t)p.k * 2u);
    uint32_t aoff[MI];
#pragma unroll
    for (int i = 0; i < MI; i++)
        aoff[i] = ((uint32_t)(by * BM + 16 * i + r16) * (uint32_t)p.k + (uint32_t)(ub + u0) * 32u + 8u * g) * 2u;

    floatx4 acc[MI][4];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    half8 fa[UMAX][MI];
    auto load_a = [&](int u) {
#pragma unroll
        for (int s = 0; s < UMAX; s++) {
            const uint32_t du = (uint32_t)(min(u + s, u1 - 1) - u0) * 64u;
#pragma unroll
            for (int i = 0; i < MI; i++) fa[s][i] = bload16<AX>(ra, aoff[i] + du);
        }
    };
    // The weight fragments of unit s + 1 are read from LDS while unit s's MFMAs run (the reads
    // are unconditional, clamped to the wave's last unit; only the MFMAs are skipped).
    auto mma = [&](int u) {
        half8 fw[2][4];
        auto rd = [&](half8 (&f)[4], int uu) {
#pragma unroll
            for (int j = 0; j < 4; j++) f[j] = *(const half8*)(wl + (uu * 4 + j) * 512 + l * 8);
        };
        rd(fw[0], u);
#pragma unroll
        for (int s = 0; s < UMAX; s++) {
            if (s + 1 < UMAX) rd(fw[(s + 1) & 1], min(u + s + 1, u1 - 1));
            if (u + s < u1) {  // wave-uniform
#pragma unroll
                for (int i = 0; i < MI; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) acc[i][j] = mfma16(fw[s & 1][j], fa[s][i], acc[i][j]);
            }
        }
    };
    if (u0 < u1) load_a(u0);
    __builtin_amdgcn_s_waitcnt(0);  // the weight tile's loads (and the first a chunk) are done
    __syncthreads();                // ... for every wave: the whole tile is in LDS
    mark(0);
    for (int u = u0; u < u1; u += UMAX) {
        if (u != u0) load_a(u);
        mma(u);
    }
    __syncthreads();  // every wave is done with the weight tile: the reduction reuses its space
    mark(1);

    float* red = (float*)lds;
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
    __syncthreads();  // LDS is free again
    mark(2);
    finish<NPASS, EPI, true>(p, v, bx * p.tiles_m + by, z, by * BM, bx, BM, s_last, ec, er);
    if (sub) {
        release_wait();
        mark(3);
    }
}

}  // namespace jh
