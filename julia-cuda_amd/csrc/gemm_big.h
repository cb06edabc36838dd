// One output tile of the throughput GEMM (BM x BN = 256 x 256 or 128 x 128), as a device function:
// the body of the per-GEMM `gemm_big` kernel for large M. c = epilogue(a . w^T) with the
// epilogues of the latency tile (device.h), applied straight from the accumulators.
//
// Waves in a 2 x (BN / 64) grid (eight for 256 x 256: two a SIMD, so that one wave's MFMAs run
// while the other waits on its copies or LDS reads) each own a (BM / 2) x 64 block of outputs,
// computed with MFMA 32 x 32 x 16 as MR = BM / 64 row fragments x 2 column fragments, w as the
// MFMA's A operand: lane l of fragment (i, c) holds output row 32 i + l % 32 and columns
// 32 c + 8 q + 4 (l / 32) + e, q, e < 4. A 256 x 256 tile reads 64 bytes of operands per
// 8 Kflop, half what a 256 x 128 tile reads: the copy path into a CU (about 64 bytes per clock)
// keeps up with the MFMAs.
//
// The K loop runs BK = 32 at a time through four LDS stages filled by direct buffer -> LDS loads
// (no register staging), three stages ahead, with one block barrier per stage. A stage's copies
// are issued between the MFMAs of the stage three back: issued in one burst they stall the
// issuing wave on the address path while its MFMA unit idles.
//  - a's stage: BM rows x 64 bytes; copy I takes rows 16 I .. 16 I + 15 (4 lanes a row), lane l
//    into LDS chunk 64 I + l, which is row r = 16 I + l / 4, chunk l % 4, and holds a's chunk
//    (l % 4) ^ ((r / 4) % 4) of that row: the 16 rows one fragment read serves per LDS cycle
//    cover all 64 banks.
//  - w's stage: BN / 64 blocks of the fragment-ordered matrix (64 columns x one 32-wide K unit,
//    4 KB contiguous each), copied as they are.
//
// The epilogue's column-wise part runs on the accumulators: a lane has MR output rows, so the row
// data (LayerNorm statistics, positions) is a few values a lane, loaded with the first stage, and
// each row's mean and rstd are computed once a tile (two threads a row) into LDS; the column
// data (colsum, bias) is loaded with the first stage into LDS; the rotate-half pair (x, x + 32) of a head and the GeGLU (input, gate) pair sit in one
// lane. The result goes through LDS into row-contiguous 16-byte pieces for the residual, the
// output statistics and the stores. The RoPE table rows and the residual are loaded two row
// fragments ahead, the first two right after the last MFMAs are issued.
#pragma once

#include "gemm_tile.h"

namespace jh {

template <int BM, int BN>
struct Big {
    static_assert((BM == 256 && BN == 256) || (BM == 192 && BN == 256) || (BM == 128 && BN == 128),
                  "tile shape");
    static constexpr int TM = BM, TN = BN, BK = 32, NSTAGE = 4;
    static constexpr int WAVES_M = 2, WAVES_N = BN / 64;  // 2 x 4 waves (BN 256) or 2 x 2 (128)
    static constexpr int NWAVES = WAVES_M * WAVES_N, THREADS = 64 * NWAVES;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;  // a wave's block
    static constexpr int MR = WM / 32, NC = WN / 32;  // its 32 x 32 fragments
    static constexpr int NG = WN / 64;                // its 64-column groups
    static constexpr int A_BYTES = BM * BK * 2, W_BYTES = BN * BK * 2;
    static constexpr int STAGE = A_BYTES + W_BYTES;   // bytes per stage
    static constexpr int NCOPY = STAGE / 1024, A_COPIES = A_BYTES / 1024;  // 1 KB copies a stage
    // Copies per wave and stage: LOADS for waves below FULL, LOADS - 1 for the rest (192 x 256:
    // 28 copies over eight waves; the square tiles: LOADS for every wave).
    static constexpr int LOADS = (NCOPY + NWAVES - 1) / NWAVES;
    static constexpr int FULL = NCOPY - (LOADS - 1) * NWAVES;
    static constexpr bool EVEN = FULL == NWAVES && A_BYTES == W_BYTES;
    static constexpr int COLS = NSTAGE * STAGE;       // per wave: colsum, bias of its columns
    static constexpr int ROWS = COLS + NWAVES * 2 * WN * 4;  // per row: LayerNorm mean, rstd
    static constexpr int POSR = ROWS + BM * 8;                // per row: RoPE position
    static constexpr int LDS_BYTES = POSR + BM * 4;
    // RoPE epilogues, after the K loop: the tile's table rows (BM x 256 bytes) in the stages'
    // space, then the f16 staging of the output rows.
    static constexpr int TABLE_BYTES = BM * 256;
    static_assert(NG == 1 && LOADS >= 2, "wave blocks of 64 columns");
    static_assert(THREADS >= 2 * BM, "two threads a row for the row statistics");
};

// The column width of the throughput tile BM rows high.
__host__ __device__ constexpr int big_bn(int bm) { return bm == 192 ? 256 : bm; }

// LayerNorm statistics slots one thread reads (two threads split a row's K / 64 slots): the big
// tiles take LayerNorm epilogues for K <= 64 * 2 * BIG_LN_SLOTS.
constexpr int BIG_LN_SLOTS = 8;

// Task `task` of tiles_n * tiles_m (x splits with SPLIT; XCD-mapped: an XCD takes a contiguous
// range of tasks, in the grouped order below). AX: a is read device-coherent; XG: the input
// statistics are read device-coherent. The outputs and output statistics are stored
// device-coherent on every path (written through the L2: a kernel's end then has no dirty lines
// of them to write back before the next kernel reads them from the other XCDs; measured at 4096
// rows, qkv 23.2 -> 21.2 µs, wo 12.3 -> 11.3, wi 24.7 -> 23.4, wo_mlp 15.8 -> 14.9, and level at
// 18752). The residual is read through the caches.
// SPLIT: p.splits K splits a tile (the instances without it keep the whole K loop's code as it
// is).
template <int BM, int BN, int EPI, bool AX, bool XG, bool SPLIT = false>
__device__ __forceinline__ void gemm_big_tile(const GemmParams& p, int task, char* lds,
                                              uint64_t* sub = nullptr) {
    auto mark = [&](int i) {  // profiling: thread 0's view of the task's stages
        if (sub && threadIdx.x == 0) sub[i] = wall_clock64();
    };
    mark(0);
    using C = Big<BM, BN>;
    constexpr int MR = C::MR, NC = C::NC, NG = C::NG;
    // A task is (tile, K split z): the splits of a tile are consecutive tasks, on one XCD.
    const int S = SPLIT ? p.splits : 1;
    const int L = xcd_task(task, p.tiles_n * p.tiles_m * S);
    const int z = L % S, t2 = L / S;
    // Groups of G row bands (about 2 MB of a): within a group the column block changes slowest,
    // so an XCD's concurrent tiles share a few w column blocks and the group's a bands, which
    // together fit its 4 MB L2 (a walk along whole row bands would cycle all of w through the
    // L2 once per band).
    const int G = max(1, (2 << 20) / (BM * p.k * 2));
    const int gsz = G * p.tiles_n, grp0 = t2 / gsz * G, in = t2 % gsz;
    const int rows_g = min(G, p.tiles_m - grp0);
    const int bx = in / rows_g, by = grp0 + in % rows_g;
    const int tid = threadIdx.x, l = tid & 63, l32 = l & 31, hi = l >> 5;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
    const int wm = w / C::WAVES_N, wn = w % C::WAVES_N;
    const int U = p.k >> 5;                        // K units of 32
    const int ub = z * U / S, nkt = (z + 1) * U / S - ub;  // this split's units = stages
    const int g0 = (bx * BN + wn * C::WN) >> 6;    // the wave's first 64-column group

    // ---- epilogue inputs that go with the first stage -----------------------------------------
    // Column data (colsum, bias of the wave's WN columns): two floats a lane, into the wave's own
    // LDS words after the stages, read back by the epilogue (no block barrier: one wave writes
    // and reads them).
    float* wcols = (float*)(lds + C::COLS) + w * 2 * C::WN;
    float2 cin[2];
    constexpr int CPL = C::WN / 64;  // columns a lane brings in per array
    static_assert(CPL == 1 || CPL == 2, "columns per lane");
    auto col_in = [&](const float* src, int a) {
        if (CPL == 2) cin[a] = *(const float2*)(src + g0 * 64 + 2 * l);
        else cin[a] = make_float2(src[g0 * 64 + l], 0.0f);
    };
    if (EPI & EPI_LN) col_in(p.colsum, 0);
    if (EPI & EPI_BIAS) col_in(p.bias, 1);
    // Row data: the LayerNorm statistics, two threads a row of the tile, thread t taking slots
    // t % 2, t % 2 + 2, ... of row t / 2 (unconditional loads, clamped, masked when summed); the
    // lane's RoPE positions.
    const int slots = p.k >> 6;
    float2 sl[BIG_LN_SLOTS];
    if (EPI & EPI_LN) {
        const int r = min(by * BM + min(tid >> 1, BM - 1), p.m - 1);
        const float* st = p.stats_in + (size_t)r * slots * 2;
#pragma unroll
        for (int u = 0; u < BIG_LN_SLOTS; u++) sl[u] = load8f<XG>(st + 2 * min(2 * u + (tid & 1), slots - 1));
    }
    // The RoPE position of row tid / 2 (an unconditional load: from the table itself when there
    // are no positions), into LDS with the row statistics.
    int rpos = 0;
    if (EPI & EPI_ROPE) {
        const int r = min(by * BM + min(tid >> 1, BM - 1), p.m - 1);
        const int v = *(const int*)(p.pos ? (const void*)(p.pos + r) : (const void*)p.rope);
        rpos = min(max(p.pos ? v : r, 0), p.rope_rows - 1);
    }

    // ---- the K loop ---------------------------------------------------------------------------
    // Stage copies: copy q of the wave's LOADS is load I = w + NWAVES q of the stage's A_BYTES / 1024
    // a loads then W_BYTES / 1024 w loads.
    // (Copies q < LOADS / 2 are a's, the rest w's: the test is on the unrolled q, no branch.)
    // (The square tiles: copies q < LOADS / 2 are a's, the rest w's, a test on the unrolled q;
    // 192 x 256: copy I is a's while I < A_COPIES, a wave-uniform test, and copies past NCOPY
    // are none.)
    static_assert(!C::EVEN || C::LOADS % 2 == 0, "half the copies a's");
    // The copies go through buffer descriptors over a and w (the host checks both fit 4 GB): a
    // lane's 32-bit offset of copy q at unit 0, computed once; unit kt adds kt * 64 bytes (a) or
    // kt * 4 KB (w) as the scalar offset. (Global copies take a 64-bit lane address and an added
    // 64-bit operation a copy: the GEMMs ran 2-6% slower with them.) Copies q past a 192-row
    // tile's NCOPY get an offset that is never used.
    const auto abuf = buffer_rsrc(p.a, (uint32_t)min((size_t)p.m * p.k * 2, (size_t)0xFFFFFFFFu));
    const auto wbuf = buffer_rsrc(p.w, (uint32_t)min((size_t)p.n * p.k * 2, (size_t)0xFFFFFFFFu));
    uint32_t coff[C::LOADS];
#pragma unroll
    for (int q = 0; q < C::LOADS; q++) {
        const int I = w + C::NWAVES * q;
        if (C::EVEN ? q < C::LOADS / 2 : I < C::A_COPIES) {
            const int r = 16 * I + (l >> 2), ch = (l & 3) ^ ((r >> 2) & 3);
            const int row = min(by * BM + r, p.m - 1);
            coff[q] = (uint32_t)(((size_t)row * p.k + ub * 32 + ch * 8) * 2);
        } else {
            const int J = I - C::A_BYTES / 1024;  // 4 KB block J / 4 = column group, part J % 4
            coff[q] = (uint32_t)((((bx * (BN / 64) + (J >> 2)) * U + ub) * 4 + (J & 3)) * 1024 + l * 16);
        }
    }
    auto issue_one = [&](int ks, int buf, int q) {
        char* st = lds + buf * C::STAGE;
        const int I = w + C::NWAVES * q;
        if (!C::EVEN && I >= C::NCOPY) return;
        if (C::EVEN ? q < C::LOADS / 2 : I < C::A_COPIES)
            lds_bdma16<AX>(abuf, coff[q], st + I * 1024, ks * 64);
        else
            lds_bdma16<false>(wbuf, coff[q], st + C::A_BYTES + (I - C::A_BYTES / 1024) * 1024, ks * 4096);
    };
    auto issue = [&](int kt, int buf) {
#pragma unroll
        for (int q = 0; q < C::LOADS; q++) issue_one(kt, buf, q);
    };
#pragma unroll
    for (int s = 0; s < C::NSTAGE - 1; s++)
        if (s < nkt) issue(s, s);

    // Column data of group j, half h, slice q (columns 64 j + 32 h + 8 q + 4 hi ..).
    auto col4 = [&](int a, int j, int h, int q) {
        return *(const float4*)(wcols + a * C::WN + 64 * j + 32 * h + 8 * q + 4 * hi);
    };

    // This wave's copies a stage: LOADS, or LOADS - 1 (a wave-uniform branch between the waits).
    const bool full_wave = C::EVEN || w < C::FULL;
    if (nkt > 2) {
        if (full_wave) wait_vmcnt<2 * C::LOADS>(); else wait_vmcnt<2 * C::LOADS - 2>();
    } else {
        if (full_wave) wait_vmcnt<C::LOADS>(); else wait_vmcnt<C::LOADS - 1>();
    }
    mark(1);  // (not in the loop: the clock read is a scalar-memory operation, and with one of
              // those outstanding the compiler waits for every LDS read at once)
    auto col_out = [&](int a) {
        if (CPL == 2) *(float2*)(wcols + a * C::WN + 2 * l) = cin[a];
        else wcols[a * C::WN + l] = cin[a].x;
    };
    if (EPI & EPI_LN) col_out(0);
    if (EPI & EPI_BIAS) col_out(1);
    // Each row's mean and rstd into LDS (read by the epilogue), once the first stage has landed:
    // its wait covers the slots, loaded before it (loads complete in order). The barrier before
    // the first fragment reads orders these writes before every wave's reads.
    float2* rows_ms = (float2*)(lds + C::ROWS);
    if (EPI & EPI_LN) {
        float S = 0.0f, Q = 0.0f;
#pragma unroll
        for (int u = 0; u < BIG_LN_SLOTS; u++) {
            const bool ok = 2 * u + (tid & 1) < slots;
            S += ok ? sl[u].x : 0.0f;
            Q += ok ? sl[u].y : 0.0f;
        }
        S = group_sum<2>(S);
        Q = group_sum<2>(Q);
        const float mean = S / (float)p.k;
        const float var = fmaxf(Q / (float)p.k - mean * mean, 0.0f);
        if ((tid & 1) == 0 && tid < 2 * BM) rows_ms[tid >> 1] = make_float2(mean, 1.0f / sqrtf(var + p.eps));
    }
    int* rows_pos = (int*)(lds + C::POSR);
    if ((EPI & EPI_ROPE) && (tid & 1) == 0 && tid < 2 * BM) rows_pos[tid >> 1] = rpos;

    floatx16 acc[MR][NC];
#pragma unroll
    for (int i = 0; i < MR; i++)
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][c][e] = 0.0f;

    // Fragments of one K-16 step: lane l takes K 16 t + 8 (l / 32) .. + 7 of the stage: a's chunk
    // 2 t + l / 32 of row 32 i + l % 32; w's row 32 c + l % 32 of the wave's columns, which in the
    // fragment order is block (the wave's first column) / 64 + c / 2, fragment 2 (c % 2) +
    // (l % 32) / 16, lane group 2 t + l / 32. Read r of a step, in the order the MFMAs use them:
    // w fragment 0, a fragment 0, the other w fragments, the other a fragments.
    half8 fa[2][MR], fw[2][NC];
    constexpr int NR = MR + NC;  // reads per step
    auto rd = [&](int stage, int t, int r) {
        const char* st = lds + (stage % C::NSTAGE) * C::STAGE;
        if (r == 1 || r > NC) {
            const int i = r == 1 ? 0 : r - NC;
            const int row = wm * C::WM + 32 * i + l32;
            fa[t][i] = *(const half8*)(st + row * 64 + (((2 * t + hi) ^ ((row >> 2) & 3)) << 4));
        } else {
            const int c = r == 0 ? 0 : r - 1;
            const int g = wn * (C::WN / 64) + (c >> 1), j = 2 * (c & 1) + (l32 >> 4);
            fw[t][c] = *(const half8*)(st + C::A_BYTES + (g * 4 + j) * 1024 + ((2 * t + hi) * 16 + (l & 15)) * 16);
        }
    };

    // Stage 0 is in (this wave's copies: the wait above; every wave's: the barrier).
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int r = 0; r < NR; r++) rd(0, 0, r);

    // Iteration s: (A) step 0's MFMAs with step 1's reads between them; (B) this wave's copies of
    // stage s + 1 done (stage s + 2's may stay in flight), then a bare barrier: every wave's are,
    // and every wave is done with stage s - 1 (its last reads fed MFMAs before the barrier);
    // (C) step 1's MFMAs with the next stage's step-0 reads and stage s + 3's copies (into stage
    // s - 1's buffer) between them. A step's fragments are read one MFMA phase before they are
    // used. (__syncthreads' release fence would wait for all of this wave's copies.)
    constexpr int NM = MR * NC, PER = C::LOADS, GAP = NM / PER;
    static_assert(GAP >= 1, "copies per K-16 step");
    // One stage. NEXT: a stage follows (wait for its copies, NEXT_LAST: they are the last ones in
    // flight); MORE: stage s + 3 exists. The stages up to nkt - 4 take every branch one way, so
    // the loop over them is straight-line code and the last three are peeled.
    auto stage_body = [&](int s, auto next_, auto next_last_, auto more_) {
        constexpr bool NEXT = decltype(next_)::value, NEXT_LAST = decltype(next_last_)::value;
        constexpr bool MORE = decltype(more_)::value;
#pragma unroll
        for (int x = 0; x < NM; x++) {
            const int i = x / NC, c = x % NC;
            __builtin_amdgcn_sched_barrier(0);
            acc[i][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fw[0][c], fa[0][i], acc[i][c], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (x < NR) rd(s, 1, x);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (NEXT) {
            if (NEXT_LAST)
                wait_vmcnt<0>();
            else if (full_wave)
                wait_vmcnt<C::LOADS>();
            else
                wait_vmcnt<C::LOADS - 1>();
            __builtin_amdgcn_s_barrier();
        }
#pragma unroll
        for (int x = 0; x < NM; x++) {
            const int i = x / NC, c = x % NC;
            __builtin_amdgcn_sched_barrier(0);
            acc[i][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fw[1][c], fa[1][i], acc[i][c], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (NEXT && x < NR) rd(s + 1, 0, x);
            if (MORE && x % GAP == GAP - 1 && x / GAP < PER) {
                __builtin_amdgcn_sched_barrier(0);
                issue_one(s + 3, (s + 3) % C::NSTAGE, x / GAP);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    int s = 0;
    for (; s + 3 < nkt; s++) stage_body(s, T_{}, F_{}, T_{});
    if (s + 2 < nkt) stage_body(s++, T_{}, F_{}, F_{});
    if (s + 1 < nkt) stage_body(s++, T_{}, T_{}, F_{});
    stage_body(s, F_{}, F_{}, F_{});
    mark(2);

    // ---- the epilogue -------------------------------------------------------------------------
    // Per row fragment i: the column-wise part (LayerNorm, bias, ReLU/GELU, RoPE, GeGLU) on the
    // accumulators, where a lane holds the RoPE and GeGLU pairs; the f32 result through the
    // wave's own LDS rows (32 rows of WO columns, padded to WO + 4 floats: 16 rows of one write
    // cover all 64 banks) into rows of 8 consecutive columns a lane; then the residual, the f16
    // rounding, the output statistics (8 lanes a 64-column group) and 16-byte stores, 16 (or 8)
    // lanes a row.
    constexpr bool GEGLU = (EPI & EPI_GEGLU) != 0;
    constexpr bool RES = (EPI & EPI_RES) && !GEGLU;
    constexpr bool ROPE = (EPI & EPI_ROPE) != 0;
    // The staging holds f32 where the residual and statistics follow (rounding after the
    // residual add), f16 otherwise (the same rounding, half the LDS traffic).
    constexpr bool H16 = !RES && !(EPI & EPI_STATS);
    constexpr int WO = GEGLU ? C::WN / 2 : C::WN;  // output columns of the wave
    constexpr int LPR = WO / 8, RPP = 64 / LPR;     // lanes a row, rows a pass
    constexpr int NPASS = 32 / RPP, PAD = WO + 4, PADH = WO + 8;
    static_assert(!ROPE || (H16 && C::TABLE_BYTES + C::NWAVES * 32 * PADH * 2 <= C::COLS),
                  "RoPE table and f16 staging in the stages' space");
    const int ncol = GEGLU ? (p.n >> 1) : p.n;
    const auto cbuf = buffer_rsrc(p.c, (uint32_t)min((size_t)p.m * ncol * 2, (size_t)0xFFFFFFFFu));
    const int col0 = (GEGLU ? g0 * 32 : g0 * 64);   // the wave's first output column
    char* stage_base = lds + (ROPE ? C::TABLE_BYTES : 0);
    float* sg = (float*)stage_base + w * 32 * PAD;
    f16* sgh = (f16*)stage_base + w * 32 * PADH;
    __syncthreads();  // every wave is done reading the stages

    // Split-K (kernels/src/gemm.rs:355-433), as the latency tile's (finish in gemm_tile.h): every
    // split stores its accumulators to the scratch ([tile][split][float4 v][thread], coherent
    // stores), waits for them, then counts its arrival; the tile's last arriver (which resets the
    // counter) sums every split's partial in split order, so the result does not depend on
    // arrival order, and runs the epilogue. The others are done with the task.
    if (SPLIT && S > 1) {
        constexpr int NV = MR * NC * 4;  // float4s a lane
        // (one buffer descriptor over the tile's partials: 16-byte coherent stores and loads)
        const auto part = buffer_rsrc(p.ws + (size_t)t2 * S * NV * C::THREADS * 4, S * NV * C::THREADS * 16);
        const uint32_t mine = (uint32_t)z * NV * C::THREADS * 16;
#pragma unroll
        for (int i = 0; i < MR; i++)
#pragma unroll
            for (int c = 0; c < NC; c++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    bstore16f(part, mine + (((i * NC + c) * 4 + q) * C::THREADS + tid) * 16,
                              make_float4(acc[i][c][4 * q], acc[i][c][4 * q + 1], acc[i][c][4 * q + 2],
                                          acc[i][c][4 * q + 3]));
        release_wait();
        __syncthreads();
        uint32_t* s_last = (uint32_t*)lds;  // the stages' space is free here
        if (tid == 0) {
            const uint32_t old = atomic_add_agent(p.counters + t2, 1u);
            const uint32_t last = old == (uint32_t)(S - 1);
            if (last) atomic_store_agent(p.counters + t2, 0u);
            *s_last = last;
        }
        __syncthreads();
        const uint32_t last = *s_last;
        __syncthreads();  // every thread has read s_last before the epilogue writes the space
        if (last == 0) return;
#pragma unroll
        for (int i = 0; i < MR; i++)
#pragma unroll
            for (int c = 0; c < NC; c++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[i][c][e] = 0.0f;
        for (int zz = 0; zz < S; zz++) {
            const uint32_t src = (uint32_t)zz * NV * C::THREADS * 16;
#pragma unroll
            for (int i = 0; i < MR; i++)
#pragma unroll
                for (int c = 0; c < NC; c++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 v4 = bload16f(part, src + (((i * NC + c) * 4 + q) * C::THREADS + tid) * 16);
                        acc[i][c][4 * q] += v4.x;
                        acc[i][c][4 * q + 1] += v4.y;
                        acc[i][c][4 * q + 2] += v4.z;
                        acc[i][c][4 * q + 3] += v4.w;
                    }
        }
    }

    // RoPE: the tile's table rows into LDS as whole lines (copy I takes rows 4 I .. 4 I + 3, 16
    // lanes a row; the 16-byte chunk c of row r is stored at chunk c ^ (r % 16), so that the 16
    // rows one read serves cover all 64 banks). A lane's own gathers would touch 32 lines a load
    // instruction, over again in every wave that shares the rows.
    // Every copy's row position is read first (one LDS round trip; a copy issued between them
    // would make the next read wait for it), then the copies go out through a descriptor over
    // the table (256 bytes a row).
    const char* table = lds;
    if (ROPE) {
        constexpr int COPIES = C::TM / 4 / C::NWAVES;
        const auto tbuf = buffer_rsrc(p.rope, (uint32_t)p.rope_rows * 256u);
        uint32_t toff[COPIES];
#pragma unroll
        for (int q = 0; q < COPIES; q++) {
            const int I = w + C::NWAVES * q, rr = 4 * I + (l >> 4), c = (l & 15) ^ (rr & 15);
            toff[q] = (uint32_t)rows_pos[rr] * 256u + c * 16;
        }
#pragma unroll
        for (int q = 0; q < COPIES; q++) lds_bdma16<false>(tbuf, toff[q], lds + (w + C::NWAVES * q) * 1024);
        wait_vmcnt<0>();
        __syncthreads();
    }

    struct RowIn {
        half8 rr[NPASS];        // residual, transposed layout
    };
    // The residual through a descriptor (32-bit offsets; the rows are clamped into it).
    [[maybe_unused]] const auto rbuf = buffer_rsrc(RES ? (p.res ? p.res : p.c) : p.c,
                                                   (uint32_t)min((size_t)p.m * ncol * 2, (size_t)0xFFFFFFFFu));
    auto load_row = [&](int i, RowIn& in) {
        if (RES) {
#pragma unroll
            for (int ps = 0; ps < NPASS; ps++) {
                const int r = min(by * BM + wm * C::WM + 32 * i + ps * RPP + l / LPR, p.m - 1);
                in.rr[ps] = bload16<false>(rbuf, ((uint32_t)r * ncol + col0 + 8 * (l % LPR)) * 2u);
            }
        }
    };
    RowIn rin[3];  // two row fragments ahead
    load_row(0, rin[0]);
    if (MR > 1) load_row(1, rin[1]);

#pragma unroll
    for (int i = 0; i < MR; i++) {
        // (scheduling fences: one row fragment's values, addresses and stores at a time)
        __builtin_amdgcn_sched_barrier(0);
        if (i + 2 < MR) load_row(i + 2, rin[(i + 2) % 3]);
        __builtin_amdgcn_sched_barrier(0);
        const RowIn& ri = rin[i % 3];
#pragma unroll
        for (int j = 0; j < NG; j++) {
            const int g = g0 + j;
            // v[h][4 q + e]: column 64 g + 32 h + 8 q + 4 hi + e
            float v[2][16];
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int x = 0; x < 16; x++) v[h][x] = acc[i][2 * j + h][x];
            if (EPI & EPI_LN) {
                const float2 ms = rows_ms[wm * C::WM + 32 * i + l32];  // (mean, rstd)
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 c4 = col4(0, j, h, q);
                        const float cc[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            v[h][4 * q + e] = ms.y * (v[h][4 * q + e] - ms.x * cc[e]);
                    }
            }
            if (EPI & EPI_BIAS) {
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 b4 = col4(1, j, h, q);
                        const float bb[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
                        for (int e = 0; e < 4; e++) v[h][4 * q + e] += bb[e];
                    }
            }
            if (EPI & EPI_RELU) {
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int x = 0; x < 16; x++) v[h][x] = fmaxf(v[h][x], 0.0f);
            }
            if (EPI & EPI_GELU) {
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int x = 0; x < 16; x++) v[h][x] = gelu(v[h][x]);
            }
            if (EPI & EPI_ROPE) {
                // q and k heads: columns x and x + 32 of a head are the rotate-half pair of
                // dimension x; the table holds (cos, sin) per dimension.
                if (g * 64 < p.rope_cols) {
                    const int tr = wm * C::WM + 32 * i + l32;  // the row in the tile
                    const char* trow = table + tr * 256;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        // dimensions 8 q + 4 hi .. + 3: chunks 4 q + 2 hi and + 1
                        const int ca = 4 * q + 2 * hi;
                        const float4 t0 = *(const float4*)(trow + ((ca ^ (tr & 15)) << 4));
                        const float4 t1 = *(const float4*)(trow + (((ca + 1) ^ (tr & 15)) << 4));
                        const float co[4] = {t0.x, t0.z, t1.x, t1.z}, sn[4] = {t0.y, t0.w, t1.y, t1.w};
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const float x1 = v[0][4 * q + e], x2 = v[1][4 * q + e];
                            v[0][4 * q + e] = x1 * co[e] - x2 * sn[e];
                            v[1][4 * q + e] = x2 * co[e] + x1 * sn[e];
                        }
                    }
                }
            }
            float* dst = sg + l32 * PAD + 4 * hi;
            f16* dsth = sgh + l32 * PADH + 4 * hi;
            if (H16 && !GEGLU) {
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        half4 o;
#pragma unroll
                        for (int e = 0; e < 4; e++) o[e] = (f16)v[h][4 * q + e];
                        *(half4*)(dsth + 64 * j + 32 * h + 8 * q) = o;
                    }
            } else if (GEGLU) {
                // Packed rows 64 g + x are the input of output column 32 g + x, + 32 its gate.
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    float4 o;
                    o.x = gelu(v[0][4 * q]) * v[1][4 * q];
                    o.y = gelu(v[0][4 * q + 1]) * v[1][4 * q + 1];
                    o.z = gelu(v[0][4 * q + 2]) * v[1][4 * q + 2];
                    o.w = gelu(v[0][4 * q + 3]) * v[1][4 * q + 3];
                    *(float4*)(dst + 32 * j + 8 * q) = o;
                }
            } else {
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        *(float4*)(dst + 64 * j + 32 * h + 8 * q) =
                            make_float4(v[h][4 * q], v[h][4 * q + 1], v[h][4 * q + 2], v[h][4 * q + 3]);
            }
        }
        // The wave's rows back, 8 columns a lane (LDS operations of one wave complete in order).
        // Lanes 8-15 of each 16 read their two halves in the other order: no two lanes of a
        // 16-lane group share a bank.
        const int cl = 8 * (l % LPR), sw = (LPR == 16 && (l & 8)) ? 4 : 0;
#pragma unroll
        for (int ps = 0; ps < NPASS; ps++) {
            const int rl = ps * RPP + l / LPR;
            half8 o;
            if (H16 && !GEGLU) {
                o = *(const half8*)(sgh + rl * PADH + cl);
            } else {
                const float* src = sg + rl * PAD + cl;
                const float4 a0 = *(const float4*)(src + sw), a1 = *(const float4*)(src + 4 - sw);
                const float4 lo = sw ? a1 : a0, hi4 = sw ? a0 : a1;
                float y[8] = {lo.x, lo.y, lo.z, lo.w, hi4.x, hi4.y, hi4.z, hi4.w};
                if (RES) {
#pragma unroll
                    for (int e = 0; e < 8; e++) y[e] += (float)ri.rr[ps][e];
                }
#pragma unroll
                for (int e = 0; e < 8; e++) o[e] = (f16)y[e];
            }
            const int row = by * BM + wm * C::WM + 32 * i + rl;
            const bool valid = row < p.m;
            // One 16-byte buffer store (device-coherent), no branch: a row past m takes an
            // offset past the descriptor's range (the host keeps the output under 0xFFFFFF00
            // bytes), and the hardware drops the store.
            bstore16<true>(cbuf, valid ? ((uint32_t)row * ncol + col0 + cl) * 2u : 0xFFFFFF00u, o);
            if (EPI & EPI_STATS) {
                float s = 0.0f, sq = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float b = (float)o[e];
                    s += b, sq += b * b;
                }
                s = group_sum<8>(s);
                sq = group_sum<8>(sq);
                if (valid && (l & 7) == 0)
                    store8<true>(p.stats_out + ((size_t)row * (p.n >> 6) + (col0 + cl) / 64) * 2, make_float2(s, sq));
            }
        }
    }
    // Every wave is done with the LDS before the block's next task (the persistent kernel runs
    // several in a row) copies into it. A bare barrier after the wave's LDS operations: the
    // tile's stores drain while the next tile's copies go out (__syncthreads would wait for
    // them; when all CUs end a round at once, their stores queue for the HBM for microseconds).
    // The next tile's stage waits count these stores too, which only makes them wait longer.
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    mark(3);
}

}  // namespace jh
