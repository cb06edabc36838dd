// One (64 queries, head, key range) tile of the attention, as a device function: the body of the
// per-layer `attention_kernel` and a task of the persistent layer kernel, which pass their own
// LDS. See attention.hip for the design.
#pragma once

#include <type_traits>

#include "device.h"

namespace jh {

constexpr int ATT_PART = 18;  // f32 per thread in a key-range partial: 16 outputs, max, sum

// Rows up to which one key range may go to the 16-query slice tile; above, the streaming tile.
constexpr int ATT_SLICE_ROWS = 2048;

// Which tile one key range takes in the persistent kernel, which compiles these two (the
// per-step kernels choose in attention_launch; measured on MI355X, one sequence, heads of 64):
// the slice tile while a query's keys are few (global attention under ~400 rows: 293 rows
// 5.2 us against 7.4; a +-64 window up to ~1500 rows: 1024 rows 5.4 against 6.0), the
// streaming tile past that (global 448 rows 9.0 us against 9.3, 1024 rows 17.1 against 21.3;
// window 2048 rows 7.2 against 9.2), where the slice tile's per-slice restaging of every key
// costs more than it saves in latency.
__host__ __device__ constexpr bool att_use_stream(int n, int window) {
    return n > ATT_SLICE_ROWS || (window == 0 ? n >= 400 : n > 1536);
}

// LDS f16 attention_tile needs: the K tile [64 keys][72] and the V^T tile [64 d][68].
constexpr int ATT_LDS_F16 = 64 * 72 + 64 * 68;

// Tile (query block qb, head h), key range `chunk` of p.chunks. Every thread of the block calls
// it; `lds` holds ATT_LDS_F16 f16 (16-byte aligned). It ends with a block barrier, so the
// caller may reuse lds right after. XG: o is read by other blocks of the same kernel (the
// persistent layer kernel), so it is stored device-coherent.
template <bool XG = false>
__device__ __forceinline__ void attention_tile(const AttnParams& p, int qb, int h, int chunk,
                                               f16* lds, uint32_t* s_last) {
    f16 (*ks)[72] = (f16 (*)[72])lds;              // [key][d], rows of 144 B
    f16 (*vt)[68] = (f16 (*)[68])(lds + 64 * 72);  // [d][key], rows of 136 B
    const int n = p.n, d = p.d, ld = 3 * d, heads = d >> 6;
    const int q0 = qb * 64;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r16 = l & 15, g = l >> 4;

    // Key blocks this tile needs, then this chunk's range of them (possibly empty). With
    // concatenated sequences (p.seg) a query sees the keys of its own sequence only: the tile's
    // keys lie between its first row's sequence start and its last row's sequence end.
    const int nb = (n + 63) >> 6;
    int kb0 = 0, kb1 = nb;
    if (p.seg) {
        kb0 = p.seg[2 * q0] >> 6;
        kb1 = ((p.seg[2 * min(q0 + 63, n - 1) + 1] - 1) >> 6) + 1;
    }
    if (p.window > 0) {
        kb0 = max(kb0, max(q0 - p.window, 0) >> 6);
        kb1 = min(kb1, (min(q0 + 63 + p.window, n - 1) >> 6) + 1);
    }
    const int nkb = kb1 - kb0;
    const int c0 = kb0 + chunk * nkb / p.chunks, c1 = kb0 + (chunk + 1) * nkb / p.chunks;

    // This wave's 16 queries as B operands (two K steps over d = 64), and each query's key
    // bounds (its sequence's rows).
    const int qi = q0 + 16 * w + r16;
    int slo = 0, shi = n;
    if (p.seg) {
        slo = p.seg[2 * min(qi, n - 1)];
        shi = p.seg[2 * min(qi, n - 1) + 1];
    }
    half8 qf[2];
    {
        const f16* qp = (const f16*)p.qkv + (size_t)min(qi, n - 1) * ld + h * 64 + 8 * g;
        qf[0] = load16h<XG>(qp);
        qf[1] = load16h<XG>(qp + 32);
        if (qi >= n) qf[0] = qf[1] = half8{};
    }

    // Staging of one key block: thread t loads K chunk (key t / 8, d chunk t % 8) and (t + 256),
    // and V chunks keyed the other way round (key t % 64, d chunk t / 64 and + 4) so that its
    // transposed LDS writes are consecutive in the key. Keys past n are zero.
    half8 kr[2], vr[2];
    uint32_t kmask[2], vmask[2];
    auto gload = [&](int kb) {
        const int base = kb * 64;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int ck = tid + 256 * u;
            const int key = base + (ck >> 3);
            // Unconditional loads (clamped rows, masked after): see the GEMM's main loop.
            kr[u] = load16h<XG>((const f16*)p.qkv + (size_t)min(key, n - 1) * ld + d + h * 64 + (ck & 7) * 8);
            const int vkey = base + (tid & 63), vch = (tid >> 6) + 4 * u;
            vr[u] = load16h<XG>((const f16*)p.qkv + (size_t)min(vkey, n - 1) * ld + 2 * d + h * 64 + vch * 8);
            kmask[u] = key < n ? 0xffffffffu : 0u;
            vmask[u] = vkey < n ? 0xffffffffu : 0u;
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int ck = tid + 256 * u;
            *(half8*)&ks[ck >> 3][(ck & 7) * 8] = mask16(kr[u], kmask[u]);
            const int vkey = tid & 63, vch = (tid >> 6) + 4 * u;
            const half8 v = mask16(vr[u], vmask[u]);
#pragma unroll
            for (int e = 0; e < 8; e++) vt[vch * 8 + e][vkey] = v[e];
        }
    };

    const float scale = 1.4426950408889634f / 8.0f;  // log2(e) / sqrt(64)
    float mx = -INFINITY, lsum = 0.0f;
    floatx4 oacc[4];
#pragma unroll
    for (int t = 0; t < 4; t++) oacc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    if (c0 < c1) gload(c0);
    for (int kb = c0; kb < c1; kb++) {
        __syncthreads();  // the previous block's tiles are no longer read
        lstore();
        __syncthreads();
        if (kb + 1 < c1) gload(kb + 1);
        const int kbase = kb * 64;

        // S^T for keys 16 t + 4 g + e of this block, query qi.
        floatx4 s[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            s[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks_ = 0; ks_ < 2; ks_++) {
                const half8 kf = *(const half8*)&ks[16 * t + r16][32 * ks_ + 8 * g];
                s[t] = mfma16(kf, qf[ks_], s[t]);
            }
        }
        float bm = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int key = kbase + 16 * t + 4 * g + e;
                const int dist = qi > key ? qi - key : key - qi;
                const bool ok = key >= slo && key < shi && (p.window == 0 || dist <= p.window);
                s[t][e] = ok ? s[t][e] * scale : -INFINITY;
                bm = fmaxf(bm, s[t][e]);
            }
        bm = max_xor32(max_xor16(bm));
        const float mnew = fmaxf(mx, bm);
        const float base = mnew == -INFINITY ? 0.0f : mnew;  // no valid key yet: exp2(-inf) = 0
        const float alpha = fast_exp2(mx - base);
        mx = mnew;
        float rs = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                s[t][e] = fast_exp2(s[t][e] - base);
                rs += s[t][e];
            }
        lsum = lsum * alpha + rs;
#pragma unroll
        for (int t = 0; t < 4; t++) oacc[t] *= alpha;

        // O^T += V^T . P^T: K step k2 covers keys 32 k2 .. 32 k2 + 31; lane group g holds keys
        // 32 k2 + 4 g + (0..3) and 32 k2 + 16 + 4 g + (0..3) (its S^T values of tiles 2 k2 and
        // 2 k2 + 1), and reads the same keys of V^T.
#pragma unroll
        for (int k2 = 0; k2 < 2; k2++) {
            half8 pf;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                pf[e] = (f16)s[2 * k2][e];
                pf[4 + e] = (f16)s[2 * k2 + 1][e];
            }
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                const half4 a = *(const half4*)&vt[16 * dt + r16][32 * k2 + 4 * g];
                const half4 b = *(const half4*)&vt[16 * dt + r16][32 * k2 + 16 + 4 * g];
                const half8 vf = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
                oacc[dt] = mfma16(vf, pf, oacc[dt]);
            }
        }
    }

    if (p.chunks > 1) {
        const int tile = qb * heads + h;
        float* slots = p.ws + (size_t)tile * p.chunks * ATT_PART * 256;
        float* mine = slots + (size_t)chunk * ATT_PART * 256 + tid;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int e = 0; e < 4; e++) xstore32(mine + (dt * 4 + e) * 256, oacc[dt][e]);
        xstore32(mine + 16 * 256, mx);
        xstore32(mine + 17 * 256, lsum);
        release_wait();
        __syncthreads();
        if (tid == 0) {
            const uint32_t old = atomic_add_agent(p.counters + tile, 1u);
            const uint32_t last = old == (uint32_t)(p.chunks - 1);
            if (last) atomic_store_agent(p.counters + tile, 0u);
            *s_last = last;
        }
        __syncthreads();
        const uint32_t last = *s_last;
        __syncthreads();  // every thread has read s_last (and is done with the tiles)
        if (last == 0) return;
        // The other ranges' partials through the coherent path (no cache invalidation).
        float m = -INFINITY;
        for (int z = 0; z < p.chunks; z++) m = fmaxf(m, xload32(slots + (size_t)z * ATT_PART * 256 + 16 * 256 + tid));
        const float base = m == -INFINITY ? 0.0f : m;
        lsum = 0.0f;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) oacc[dt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int z = 0; z < p.chunks; z++) {
            const float* src = slots + (size_t)z * ATT_PART * 256 + tid;
            const float f = fast_exp2(xload32(src + 16 * 256) - base);
            lsum += xload32(src + 17 * 256) * f;
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int e = 0; e < 4; e++) oacc[dt][e] += xload32(src + (dt * 4 + e) * 256) * f;
        }
    }

    const float tot = sum_xor32(sum_xor16(lsum));
    const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;
    if (qi < n) {
        f16* op = (f16*)p.o + (size_t)qi * d + h * 64 + 4 * g;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            half4 o;
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = (f16)(oacc[dt][e] * inv);
            store8<XG>(op + 16 * dt, o);
        }
    }
    __syncthreads();  // the tiles are free again
}

// ---- the LDS-resident query slice ---------------------------------------------------------
// The same arithmetic as attention_tile, shaped for latency: a task is 16 queries of one head
// (n / 16 x heads tasks, so short sequences still spread over the GPU), and the block's four
// waves split the slice's key range between them in steps of 32 keys, each keeping its own
// running max, sum and output, merged through LDS at the end. Q and the key range's K and V go
// into LDS with direct global -> LDS loads, all in one round trip (ranges longer than `gkeys`
// keys go in groups). K and V stay row-major ([key][d], 128-byte rows, the 16-byte chunks of row
// r stored at chunk ^ (r % 8) so a fragment's 16 rows spread over the banks); V^T fragments come
// from the transposing LDS read. No key ranges across blocks.

// LDS bytes of attention_slice_tile staging up to gkeys keys at once (a multiple of 32) with nw
// waves; the waves' merge reuses the space.
__host__ __device__ constexpr int att_lds_bytes(int gkeys, int nw = 4) {
    return 2048 + 256 * gkeys > nw * 18 * 64 * 4 ? 2048 + 256 * gkeys : nw * 18 * 64 * 4;
}

// Byte offset of 16-byte chunk `ch` of row `r` in a swizzled [rows][64 f16] LDS tile.
__device__ __forceinline__ int att_swz(int r, int ch) { return (r * 8 + (ch ^ (r & 7))) * 16; }

// Task `task` of (n + 15) / 16 slices x heads (XCD-mapped so a head's slices share an XCD's L2),
// by a block of NW waves. XL: qkv is read device-coherent; XS: o is stored device-coherent.
template <bool XL = false, bool XS = false, int NW = 4>
__device__ __forceinline__ void attention_slice_tile(const AttnParams& p, int task, char* lds,
                                                     int gkeys, uint64_t* sub = nullptr) {
    auto mark = [&](int i) {  // profiling: thread 0's view of the task's stages
        if (sub && threadIdx.x == 0) sub[i] = wall_clock64();
    };
    const int n = p.n, d = p.d, ld = 3 * d, heads = d >> 6;
    const int slices = (n + 15) >> 4, T = slices * heads;
    const int L = xcd_task(task, T);
    const int h = L / slices, q0 = (L % slices) * 16;
    const int tid = threadIdx.x, l = tid & 63, r16 = l & 15, g = l >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int j = r16 >> 2, q = r16 & 3;
    char* qs = lds;
    char* ks = lds + 2048;
    char* vs = ks + gkeys * 128;

    // The keys any of the 16 queries may see: their sequences' rows (all n rows, or from the
    // first query's sequence start to the last query's sequence end), cut to the window.
    const int qlast = min(q0 + 15, n - 1);
    int k0 = p.seg ? p.seg[2 * q0] : 0, k1 = p.seg ? p.seg[2 * qlast + 1] : n;
    if (p.window > 0) {
        k0 = max(k0, q0 - p.window);
        k1 = min(k1, q0 + 16 + p.window);
    }
    k0 &= ~31;

    // rows [r0, r0 + rows) (rows % 8 == 0) of qkv's columns col .. col + 63, clamped to row
    // n - 1, into `dst`: wave load I fills LDS chunks 64 I .. 64 I + 63, lane l chunk 64 I + l,
    // which is row c / 8, logical chunk (c % 8) ^ (row % 8).
    auto stage = [&](char* dst, int r0, int rows, int col) {
        for (int I = w; I * 64 < rows * 8; I += NW) {
            const int c = I * 64 + l, row = c >> 3, ch = (c & 7) ^ (row & 7);
            const f16* src = (const f16*)p.qkv + (size_t)min(r0 + row, n - 1) * ld + col + ch * 8;
            lds_dma16<XL>(src, dst + I * 1024);
        }
    };

    const int qi = q0 + r16;  // this lane's query (the same 16 in every wave)
    // Its own sequence's rows (keys outside are masked), and whether all 16 queries share one.
    int slo = 0, shi = n;
    if (p.seg) {
        const int qc = min(qi, n - 1);
        slo = p.seg[2 * qc], shi = p.seg[2 * qc + 1];
    }
    const bool one_seq = !p.seg || p.seg[2 * q0] == p.seg[2 * qlast];
    const int ulo = p.seg ? p.seg[2 * q0] : 0, uhi = p.seg ? p.seg[2 * qlast + 1] : n;  // uniform
    // The lane's valid keys: its sequence cut to the window, [klo, khi).
    const int wl = p.window > 0 ? p.window : (1 << 30);
    const int klo = max(slo, qi - wl), khi = min(shi, qi + wl + 1);
    const uint32_t kspan = khi > klo ? (uint32_t)(khi - klo) : 0u;
    const float scale = 1.4426950408889634f / 8.0f;  // log2(e) / sqrt(64)
    float mx = -INFINITY, lsum = 0.0f;
    floatx4 oacc[4];
#pragma unroll
    for (int t = 0; t < 4; t++) oacc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    half8 qf[2];

    for (int gk = k0; gk < k1; gk += gkeys) {
        const int steps = (min(gkeys, k1 - gk) + 31) >> 5;
        if (gk == k0) stage(qs, q0, 16, h * 64);
        stage(ks, gk, steps * 32, d + h * 64);
        stage(vs, gk, steps * 32, 2 * d + h * 64);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // the group is in LDS
        if (gk == k0) {
            mark(0);
#pragma unroll
            for (int k2 = 0; k2 < 2; k2++) qf[k2] = *(const half8*)(qs + att_swz(r16, 4 * k2 + g));
        }
        for (int st = w * steps / NW; st < (w + 1) * steps / NW; st++) {
            const int kb = gk + 32 * st, rb = 32 * st;  // the step's first key and LDS row
            // Every LDS read of the step first (K fragments of its two 16-key S tiles; V^T
            // fragments: lane (g, 4 j + q) addresses key rb + 4 g + j (+ 16), d 16 dt + 4 q), so
            // their latencies overlap.
            half8 kf[2][2];
            half4 vlo[4], vhi[4];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int k2 = 0; k2 < 2; k2++)
                    kf[t][k2] = *(const half8*)(ks + att_swz(rb + 16 * t + r16, 4 * k2 + g));
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                const int ch = 2 * dt + (q >> 1), off = (q & 1) * 8;
                vlo[dt] = lds_read_tr16(vs + att_swz(rb + 4 * g + j, ch) + off);
                vhi[dt] = lds_read_tr16(vs + att_swz(rb + 16 + 4 * g + j, ch) + off);
            }
            __builtin_amdgcn_sched_barrier(0);
            // S^T for keys kb + 16 t + 4 g + e, query qi.
            floatx4 sc[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                sc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int k2 = 0; k2 < 2; k2++) sc[t] = mfma16(kf[t][k2], qf[k2], sc[t]);
            }
            // A step inside the queries' one sequence and, for all 16, inside the window needs no
            // mask.
            const bool full = one_seq && kb >= ulo && kb + 32 <= uhi &&
                              (p.window == 0 || (q0 + 15 - kb <= p.window && kb + 31 - q0 <= p.window));
            float bm = -INFINITY;
            if (full) {
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        bm = fmaxf(bm, sc[t][e]);
                    }
            } else {
                // key kb + 16 t + 4 g + e is valid iff it lies in [klo, khi)
                const int base = kb + 4 * g - klo;
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const bool ok = (uint32_t)(base + 16 * t + e) < kspan;
                        sc[t][e] = ok ? sc[t][e] : -INFINITY;
                        bm = fmaxf(bm, sc[t][e]);
                    }
            }
            bm = max_xor32(max_xor16(bm)) * scale;  // the scores stay unscaled until the exponent
            const float mnew = fmaxf(mx, bm);
            const float base = mnew == -INFINITY ? 0.0f : mnew;  // no valid key yet: exp2(-inf) = 0
            const float alpha = fast_exp2(mx - base);
            mx = mnew;
            float rs = 0.0f;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    sc[t][e] = fast_exp2(fmaf(sc[t][e], scale, -base));
                    rs += sc[t][e];
                }
            lsum = lsum * alpha + rs;
            // O^T += V^T . P^T: lane group g holds (as its P^T values) keys kb + 4 g + (0..3) and
            // kb + 16 + 4 g + (0..3), the keys of its V^T fragment.
            half8 pf;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                pf[e] = (f16)sc[0][e];
                pf[4 + e] = (f16)sc[1][e];
            }
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                const half4 lo = vlo[dt], hi = vhi[dt];
                const half8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                oacc[dt] = mfma16(vf, pf, oacc[dt] * alpha);  // rescaled to the new max
            }
        }
        __syncthreads();  // the group's tiles are no longer read
    }

    // The waves' partials (output, max, sum over the query's keys) through LDS; then every wave
    // merges 16 / NW of the lane's 16 output values (over the partials in wave order).
    const float tot = sum_xor32(sum_xor16(lsum));
    float* mg = (float*)lds;  // [wave][18][64]
    static_assert(NW == 4 || NW == 8, "waves");
    constexpr int VPW = 16 / NW;  // output values a wave merges: dt = f / 4, e = f % 4
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int e = 0; e < 4; e++) mg[(w * 18 + dt * 4 + e) * 64 + l] = oacc[dt][e];
    mg[(w * 18 + 16) * 64 + l] = mx;
    mg[(w * 18 + 17) * 64 + l] = tot;
    __syncthreads();
    {
        float m = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < NW; ww++) m = fmaxf(m, mg[(ww * 18 + 16) * 64 + l]);
        const float base = m == -INFINITY ? 0.0f : m;
        float sum = 0.0f, o[VPW];
#pragma unroll
        for (int v = 0; v < VPW; v++) o[v] = 0.0f;
        const int f0 = w * VPW;  // the wave's first value
#pragma unroll
        for (int ww = 0; ww < NW; ww++) {
            const float f = fast_exp2(mg[(ww * 18 + 16) * 64 + l] - base);
            sum += mg[(ww * 18 + 17) * 64 + l] * f;
#pragma unroll
            for (int v = 0; v < VPW; v++) o[v] += mg[(ww * 18 + f0 + v) * 64 + l] * f;
        }
        mark(1);
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        if (qi < n) {
            // value f0 + v is dimension 16 (f / 4) + 4 g + f % 4 of query qi
            f16* op = (f16*)p.o + (size_t)qi * d + h * 64 + 4 * g + 16 * (f0 >> 2) + (f0 & 3);
            if (VPW == 4) {
                half4 ov;
#pragma unroll
                for (int v = 0; v < 4; v++) ov[v] = (f16)(o[v] * inv);
                store8<XS>(op, ov);
            } else {
                half2 ov;
                ov[0] = (f16)(o[0] * inv);
                ov[1] = (f16)(o[VPW > 1 ? 1 : 0] * inv);
                store4<XS>(op, ov);
            }
        }
        if (sub) {
            release_wait();
            mark(2);
        }
    }
    __syncthreads();  // LDS is free again
}

// ---- the streaming tile: long concatenated inputs ---------------------------------------------
// A task is (16 NW queries, head): each of the NW waves runs the online softmax over every key of
// the tile's range for its own 16 queries (no merge between waves). The key range (cut to the
// rows' sequences and the window) goes through two LDS stages of 64 keys, K and V row-major and
// swizzled as in the slice tile, filled by direct global -> LDS loads one block ahead of the
// MFMAs; a 64-key block is two of the slice tile's 32-key steps. Each key is read once per 64
// queries, and with four blocks a CU (32 KB of LDS and 108 registers a lane each) the waves
// hide each other's step latencies.
//
// KS = 2 or 4 (one long sequence, a grid of about a block a CU): the block has KS groups of NW
// waves, each running the online softmax of the same NW x 16 queries over every KS-th key
// block (group g takes blocks g, g + KS, ...) through its own stage ring, in lockstep (one
// block barrier a step for all); groups 1 .. KS - 1 then pass their running max, sum and
// output through LDS and group 0 merges them (in group order: deterministic). Two or four
// waves a SIMD instead of one hide each other's step latencies where the grid leaves the CUs
// a block each, and the chain of steps is KS times shorter. NW = 1, KS = 4 (short inputs: a
// task per 16-query slice and head, the grid about a block a CU): four single-wave groups, each
// issuing all 16 copies of its stages, so a slice's few key blocks are spread over four waves.
constexpr int ATT_STREAM_STAGES = 2;
constexpr int ATT_STREAM_LDS = ATT_STREAM_STAGES * 16384;

// One 64-key block of the streaming tile for a wave's 16 queries (lane l: query l % 16): S^T for
// keys kb + 16 t + 4 g + e (t < 4) from the block's K fragments, one max and one rescale, P . V in
// two K-32 halves. full: every score is valid; else key kb + 16 t + 4 g + e is valid iff
// (uint32_t)(base + 16 t + e) < kspan, base = kb + 4 g - (the lane's first valid key).
__device__ __forceinline__ void att_stream_block(const half8 (&kf)[4][2], const half4 (&vlo)[2][4],
                                                 const half4 (&vhi)[2][4], const half8 (&qf)[2],
                                                 bool full, int base, uint32_t kspan, float& mx,
                                                 float& lsum, floatx4 (&oacc)[4]) {
    const float scale = 1.4426950408889634f / 8.0f;  // log2(e) / sqrt(64)
    floatx4 sc[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        sc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k2 = 0; k2 < 2; k2++) sc[t] = mfma16(kf[t][k2], qf[k2], sc[t]);
    }
    float bm = -INFINITY;
    if (full) {
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                bm = fmaxf(bm, sc[t][e]);
            }
    } else {
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const bool ok = (uint32_t)(base + 16 * t + e) < kspan;
                sc[t][e] = ok ? sc[t][e] : -INFINITY;
                bm = fmaxf(bm, sc[t][e]);
            }
    }
    bm = max_xor32(max_xor16(bm)) * scale;  // the scores stay unscaled until the exponent
    const float mnew = fmaxf(mx, bm);
    const float b0 = mnew == -INFINITY ? 0.0f : mnew;  // no valid key yet: exp2(-inf) = 0
    const float alpha = fast_exp2(mx - b0);
    // The output needs rescaling only where a lane's max rose (alpha < 1): skipped when no lane
    // of the wave has (a wave-uniform test).
    const bool rescale = __builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0;
    mx = mnew;
    float rs = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            sc[t][e] = fast_exp2(fmaf(sc[t][e], scale, -b0));
            rs += sc[t][e];
        }
    lsum = lsum * alpha + rs;
    if (rescale) {
#pragma unroll
        for (int dt = 0; dt < 4; dt++) oacc[dt] = oacc[dt] * alpha;
    }
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
        half8 pf;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            pf[e] = (f16)sc[2 * hf][e];
            pf[4 + e] = (f16)sc[2 * hf + 1][e];
        }
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            const half4 lo = vlo[hf][dt], hi = vhi[hf][dt];
            const half8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            oacc[dt] = mfma16(vf, pf, oacc[dt]);
        }
    }
}

// Task `task` of (n + 16 NW - 1) / (16 NW) query blocks x heads (XCD-mapped); `lds`:
// KS x ATT_STREAM_LDS bytes; 64 NW KS threads. XS: o is stored device-coherent (the persistent
// kernel). Ends with a block barrier.
template <bool XS = false, int NW = 4, int KS = 1>
__device__ __forceinline__ void attention_stream_tile(const AttnParams& p, int task, char* lds) {
    static_assert(KS == 1 || KS == 2 || KS == 4, "key groups");
    constexpr int NS = ATT_STREAM_STAGES, QB = 16 * NW;
    constexpr int LOADS = 16 / NW;  // 1 KB copies a wave per stage
    static_assert(NW == 1 || NW == 2 || NW == 4 || NW == 8, "waves");
    const int n = p.n, d = p.d, ld = 3 * d, heads = d >> 6;
    const int tiles = (n + QB - 1) / QB;
    const int L = xcd_task(task, tiles * heads);
    const int h = L / tiles, q0 = (L % tiles) * QB;
    const int tid = threadIdx.x, l = tid & 63, r16 = l & 15, g = l >> 4;
    const int wk = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int w = wk % NW, kg = wk / NW;  // the wave's queries, its key group
    char* const ring = lds + kg * ATT_STREAM_LDS;
    const int j = r16 >> 2, q = r16 & 3;

    // The sequence bounds the tile needs, all loaded in one round trip (each costs about a
    // microsecond under load; outside the window layers' early copy below, the first copy waits
    // for them): the tile's first row's sequence start and last row's sequence end, the wave's
    // first and last rows' sequences (uniform: scalar loads), this lane's query's sequence.
    const int qlast = min(q0 + QB - 1, n - 1);
    const int wq0 = min(q0 + 16 * w, n - 1), wql = min(q0 + 16 * w + 15, n - 1);
    const int qi = q0 + 16 * w + r16;
    const int qc = min(qi, n - 1);
    // The tile's keys: from its first row's sequence start to its last row's sequence end, cut
    // to the window; 64-aligned blocks. In window layers the range starts at q0 - window
    // whatever the sequences (keys before the tile's sequence are masked like any others, and a
    // wave skips blocks wholly outside its queries' reach), so that with one key group the first
    // block's copy goes out before the bounds arrive.
    int k0 = p.window > 0 ? max(0, q0 - p.window) & ~63 : 0, k1 = n;
    int ulo = 0, uhi = n, slo = 0, shi = n;
    bool one_seq = true;
    const bool spec = KS == 1 && p.window > 0 && p.seg;  // the first copy before the bounds
    // Block b (keys k0 + 64 b ..) into stage st = b % NS: 16 wave loads of 1 KB (8 rows of K,
    // then of V), LOADS a wave; lane l fills LDS chunk 64 I + l = row c / 8, logical chunk
    // (c % 8) ^ (row % 8). The copies go through a buffer descriptor over the block's rows: the
    // lane's offsets within a block are fixed (computed once), and rows past n read as zeros
    // (their keys are masked).
    uint32_t doff[LOADS];
#pragma unroll
    for (int qq = 0; qq < LOADS; qq++) {
        const bool kk = qq < LOADS / 2;  // the first half of a wave's copies are K's
        const int I = (w + NW * qq) & 7;
        const int c = I * 64 + l, row = c >> 3, ch = (c & 7) ^ (row & 7);
        doff[qq] = (uint32_t)((row * ld + (kk ? d : 2 * d) + h * 64 + ch * 8) * 2);
    }
    auto stage = [&](int b, int st) {
        char* dst = ring + st * 16384;
        const int kb = k0 + 64 * b;
        const auto rs = buffer_rsrc((const f16*)p.qkv + (size_t)kb * ld,
                                    (uint32_t)(min(n - kb, 64) * ld * 2));
#pragma unroll
        for (int qq = 0; qq < LOADS; qq++) {
            const bool kk = qq < LOADS / 2;
            const int I = (w + NW * qq) & 7;
            lds_bdma16<false>(rs, doff[qq], dst + (kk ? 0 : 8192) + I * 1024);
        }
    };
    if (spec) stage(0, 0);
    if (p.seg) {
        const int t0 = p.seg[2 * q0], t1 = p.seg[2 * qlast + 1];
        const int w0 = p.seg[2 * wq0], wls = p.seg[2 * wql], wle = p.seg[2 * wql + 1];
        const int2 sq = *(const int2*)(p.seg + 2 * qc);
        if (p.window == 0) k0 = t0 & ~63;
        k1 = t1, ulo = w0, uhi = wle, one_seq = w0 == wls, slo = sq.x, shi = sq.y;
    }
    if (p.window > 0) k1 = min(k1, q0 + QB + p.window);
    const int nblk = k1 > k0 ? (k1 - k0 + 63) >> 6 : 0;

    // This lane's valid keys: its sequence cut to the window, [klo, khi).
    const int wl = p.window > 0 ? p.window : (1 << 30);
    const int klo = max(slo, qi - wl), khi = min(shi, qi + wl + 1);
    const uint32_t kspan = khi > klo ? (uint32_t)(khi - klo) : 0u;
    // Keys any of the wave's 16 queries may see, [wlo, whi): the wave skips the MFMAs and the
    // softmax of a block wholly outside (every score masked: the step would change nothing).
    const int wlo = __builtin_amdgcn_readfirstlane(max(ulo, wq0 - wl));
    const int whi = __builtin_amdgcn_readfirstlane(min(uhi, wql + wl + 1));
    half8 qf[2];
    {
        const f16* qp = (const f16*)p.qkv + (size_t)qc * ld + h * 64 + 8 * g;
        qf[0] = load16h<false>(qp);
        qf[1] = load16h<false>(qp + 32);
    }

    float mx = -INFINITY, lsum = 0.0f;
    floatx4 oacc[4];
#pragma unroll
    for (int t = 0; t < 4; t++) oacc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    // The lane's LDS offsets within a stage, loop-invariant: with the stage a constant in each
    // unrolled step below, every read is a base register plus an immediate. (Rows 16 t, and
    // 32 hf + 16 x, keep the swizzle of their row % 8: offsets 2048 t, 4096 hf + 2048 x.)
    int koff[2], voff[4];
#pragma unroll
    for (int k2 = 0; k2 < 2; k2++) koff[k2] = att_swz(r16, 4 * k2 + g);
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
        voff[dt] = 8192 + att_swz(4 * g + j, 2 * dt + (q >> 1)) + (q & 1) * 8;

    // The group's step b: its block kg + KS b (if there is one), in stage ST = b % NS (a
    // constant). Both groups take every step: the barrier is the block's. A step waits for its
    // block's copies (the only ones in flight), issues every LDS read of the block, then copies
    // the next block into the other stage and computes while that copy flies: the compiler
    // makes any LDS read wait for every direct-to-LDS copy in flight (it cannot tell the stages
    // apart), so a copy issued before a read would be waited for there.
    const int nsteps = (nblk + KS - 1) / KS;
    auto has = [&](int b) { return kg + KS * b < nblk; };
    auto step = [&](int b, auto st_) {
        constexpr int ST = decltype(st_)::value;
        // This wave's copies of the block done, then every wave's: and every wave is done with
        // step b - 1, whose stage step b + 1 takes.
        wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        const int kb = k0 + 64 * (kg + KS * b);
        const bool act = has(b) && !(kb + 64 <= wlo || kb >= whi);
        const char* st = ring + ST * 16384;
        // The 64 keys in one step: S^T for keys kb + 16 t + 4 g + e (t < 4), one max and one
        // rescale; P . V in two K-32 halves.
        half8 kf[4][2];
        half4 vlo[2][4], vhi[2][4];
        if (act) {
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int k2 = 0; k2 < 2; k2++) kf[t][k2] = *(const half8*)(st + koff[k2] + 2048 * t);
#pragma unroll
            for (int hf = 0; hf < 2; hf++)
#pragma unroll
                for (int dt = 0; dt < 4; dt++) {
                    vlo[hf][dt] = lds_read_tr16(st + voff[dt] + 4096 * hf);
                    vhi[hf][dt] = lds_read_tr16(st + voff[dt] + 4096 * hf + 2048);
                }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (has(b + 1)) stage(kg + KS * (b + 1), (ST + 1) % NS);
        __builtin_amdgcn_sched_barrier(0);
        if (!act) return;
        const bool full = one_seq && kb >= ulo && kb + 64 <= uhi &&
                          (p.window == 0 || (wql - kb <= p.window && kb + 63 - wq0 <= p.window));
        att_stream_block(kf, vlo, vhi, qf, full, kb + 4 * g - klo, kspan, mx, lsum, oacc);
    };

    static_assert(NS == 2, "the loop below is unrolled by the stages");
    if (has(0) && !spec) stage(kg, 0);  // (with `spec`, block 0's copy is out already)
    for (int b = 0; b < nsteps; b += NS) {
        step(b, std::integral_constant<int, 0>{});
        if (b + 1 < nsteps) step(b + 1, std::integral_constant<int, 1>{});
    }

    if (KS > 1) {
        // Groups 1 .. KS - 1: running max, sum and unnormalised output into the first rings
        // (every wave is done with the stages: the barrier); group 0 merges them with its own,
        // in group order (deterministic).
        auto slot = [&](int k) { return (float*)lds + (size_t)((k - 1) * NW + w) * 18 * 64; };
        __syncthreads();
        if (kg > 0) {
            float* mg = slot(kg);
            mg[16 * 64 + l] = mx;
            mg[17 * 64 + l] = lsum;
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int e = 0; e < 4; e++) mg[(4 * dt + e) * 64 + l] = oacc[dt][e];
        }
        __syncthreads();
        if (kg > 0) return;  // (their threads take no further barrier)
        float mk[KS];
        mk[0] = mx;
#pragma unroll
        for (int k = 1; k < KS; k++) mk[k] = slot(k)[16 * 64 + l];
        float m = mx;
#pragma unroll
        for (int k = 1; k < KS; k++) m = fmaxf(m, mk[k]);
        const float base = m == -INFINITY ? 0.0f : m;
        const float a0 = fast_exp2(mx - base);
        lsum = lsum * a0;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) oacc[dt] = oacc[dt] * a0;
#pragma unroll
        for (int k = 1; k < KS; k++) {
            const float* mg = slot(k);
            const float ak = fast_exp2(mk[k] - base);
            lsum += mg[17 * 64 + l] * ak;
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int e = 0; e < 4; e++) oacc[dt][e] += mg[(4 * dt + e) * 64 + l] * ak;
        }
    }

    const float tot = sum_xor32(sum_xor16(lsum));
    const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;
    if (qi < n) {
        f16* op = (f16*)p.o + (size_t)qi * d + h * 64 + 4 * g;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            half4 ov;
#pragma unroll
            for (int e = 0; e < 4; e++) ov[e] = (f16)(oacc[dt][e] * inv);
            store8<XS>(op + 16 * dt, ov);
        }
    }
    if (KS == 1) __syncthreads();  // LDS is free again (KS > 1: the caller's kernel ends here)
}

}  // namespace jh
