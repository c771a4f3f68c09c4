// Backward kernels of the fused PLE path (gfx950).
//
// dx[n,f]  = iw_k <g, q(W[f,phys(k)])> (+ iw_{k-1} <g, q(W[f,k-1])> when
//            k > 0 and x == e_k)                  reference backward_cuda.cu:380-490
// dW[f,phys(k)] = sum_{bin=k} q(frac) g + sum_{bin>k} g
//                                                 reference backward_cuda.cu:170-336,889-923
// db[f]    = sum_n g                              (autograd of module.py:238-239)
//
// Main path, ple_bwd_fused_kernel: one pass over grad_output.  A workgroup
// owns FS features and a chunk of samples, and walks the chunk in sub-tiles
// of P (sample, feature) pairs.  Per sub-tile it
//   A. reads the bin index and x of every pair (coalesced along the group's
//      features), computes q(frac) and the edge flag;
//   B-D. counting-sorts the pairs by (feature, bin): per 64-pair block, ranks
//      of equal keys from 64-bit ballots, a per-key prefix over blocks and a
//      block-wide scan over keys -- deterministic and stable;
//   F. lets lane groups (D/VEC lanes, one row of grad_output per step) walk
//      equal slices of the sorted rows: each row is read once, its dx is the
//      lane group's shuffle-reduced dot with the LDS weight row, and bucket /
//      weighted / bias sums run in registers until the key changes.  A slice's
//      first key goes to a per-slice record, every later key is added straight
//      into the LDS histogram (no other slice can own it);
//   G. adds the records, run by run in slice order, into the histogram;
//   H. stores dx.
// The chunk's histogram is written once; ple_bwd_finalize_kernel sums the
// chunks in chunk order and takes the suffix over bins.  No floating-point
// atomics anywhere, a fixed order for every sum, so results repeat bitwise.
//
// Fallback (shapes whose tables do not fit LDS): ple_bwd_simple_dx_kernel and
// ple_bwd_simple_hist_kernel, same partial layout, same finalize.

#include <stdlib.h>

#include "ple_device.h"
#include "ple_internal.h"

namespace ple {
namespace {

struct BwdArgs {
    const void *g;
    const float *x;
    const float *edges;
    const float *iw;
    const int32_t *nbins;
    const float *weight;
    const void *idx;
    float *dx;
    float *dw;
    float *db;
    float *part;     // [C][F][B][2D] chunk partials {bucket | weighted}
    float *part_db;  // [C][F][D] chunk partials of the bias gradient
    int64_t N;
    int F, B, D;
    int C;           // chunks in the grid (fused: a multiple of kNumXcd)
    int Cd;          // chunks holding samples (the ones that write partials)
    int64_t NC;      // samples per chunk
    int db_from_buckets;   // finalize: db = sum of the bin buckets (no raw-gradient partials)
    // fused path
    int FS, G, NT, P, LGW, nbits;   // P: pairs per sub-tile (kP)
    int o_qw, o_hist, o_db, o_edge, o_iw, o_nb, o_info, o_order, o_rank, o_cnt, o_seg, o_dx, o_rec,
        o_rkey, o_rfl, o_tmp;
};

// A row of zeros in device memory: padding rows and idle lanes of the fused
// kernel load from here, so their contributions are exact zeros without any
// masking in the row loop.  Never written.
__device__ __attribute__((aligned(16))) float g_zero_row[64] = {};

// Exclusive prefix sum of a[0..n) in place, all kBlock threads.
__device__ void block_exclusive_scan(int *a, int n, int *tmp) {
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wv = tid / kWave;
    const int per = (n + kBlock - 1) / kBlock;
    const int b0 = min(n, tid * per);
    const int b1 = min(n, b0 + per);
    int local = 0;
    for (int i = b0; i < b1; ++i) local += a[i];
    int v = local;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int t = __shfl_up(v, off);
        if (lane >= off) v += t;
    }
    if (lane == kWave - 1) tmp[wv] = v;
    __syncthreads();
    int run = v - local;
    for (int w = 0; w < wv; ++w) run += tmp[w];
    for (int i = b0; i < b1; ++i) {
        const int t = a[i];
        a[i] = run;
        run += t;
    }
    __syncthreads();
}

constexpr int kP = 1024;                        // (sample, feature) pairs per sub-tile
constexpr int kPairsPerThread = kP / kBlock;
constexpr int kRowRegs = 32;                    // gradient floats per lane in one prefetch batch (phase F)

template <int GD, int Q, int VEC, int LGW_T, typename IdxT>
__global__ __launch_bounds__(kBlock) void ple_bwd_fused_kernel(BwdArgs a) {
    constexpr int kUB = VEC == 8 ? kRowRegs / 8 : 8;   // sorted rows per prefetch batch
    // With fp32 rounding the bias gradient is the sum of the bin buckets
    // (taken at finalize); otherwise it needs its own sum of the unrounded
    // gradient.
    constexpr bool kRawDb = Q != PLE_DTYPE_F32;
    extern __shared__ __align__(16) unsigned char lds[];
    const int FS = a.FS, B = a.B, D = a.D, F = a.F, NT = a.NT;
    const int KB = B + 1;                   // keys per feature; key B marks padding rows
    float *s_qw = reinterpret_cast<float *>(lds + a.o_qw);        // [FS][B][D]
    float *s_hist = reinterpret_cast<float *>(lds + a.o_hist);    // [FS][B][2D]
    float *s_db = reinterpret_cast<float *>(lds + a.o_db);        // [FS][D]
    float *s_edge = reinterpret_cast<float *>(lds + a.o_edge);    // [FS][B+1]
    float *s_iw = reinterpret_cast<float *>(lds + a.o_iw);        // [FS][B]
    int *s_nb = reinterpret_cast<int *>(lds + a.o_nb);            // [FS]
    float2 *s_info = reinterpret_cast<float2 *>(lds + a.o_info);  // [P] {q(frac), key|edge}
    uint2 *s_sdesc = reinterpret_cast<uint2 *>(lds + a.o_order);        // [P] sorted rows {q(frac), key|edge|s<<16}
    uint8_t *s_rank = reinterpret_cast<uint8_t *>(lds + a.o_rank);      // [P]
    uint16_t *s_cnt = reinterpret_cast<uint16_t *>(lds + a.o_cnt);      // [P/64][B+1]
    int *s_seg = reinterpret_cast<int *>(lds + a.o_seg);                // [FS*(B+1)]
    float *s_dx = reinterpret_cast<float *>(lds + a.o_dx);              // [P]
    float *s_rec = reinterpret_cast<float *>(lds + a.o_rec);            // [LG][3D]
    int *s_rkey = reinterpret_cast<int *>(lds + a.o_rkey);              // [LG]
    int *s_rfl = reinterpret_cast<int *>(lds + a.o_rfl);                // [LG]
    int *s_tmp = reinterpret_cast<int *>(lds + a.o_tmp);                // [kWavesPerBlock]

    int g, c;
    if (!decode_tile(blockIdx.x, a.G, a.C, g, c)) return;
    const int f0 = g * FS;
    const int nfh = min(FS, F - f0);
    const int64_t n_begin = static_cast<int64_t>(c) * a.NC;
    const int64_t n_end = min(a.N, n_begin + a.NC);
    if (n_begin >= n_end) return;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;

    // pair inputs of a sub-tile, prefetched into registers one sub-tile ahead:
    // thread -> pairs i = tid + u * kBlock, i -> (sample i / FS, feature i % FS)
    int pk[kPairsPerThread];
    float pv[kPairsPerThread];
    auto fetch_pairs = [&](int64_t sub) __attribute__((always_inline)) {
        const int64_t ns = min(static_cast<int64_t>(NT), n_end - sub);
#pragma unroll
        for (int u = 0; u < kPairsPerThread; ++u) {
            const int i = tid + u * kBlock;
            const int s = i / FS;
            const int fl = i - s * FS;
            // unconditional loads (pair 0 stands in for padding) keep the
            // wait for them a single counted one
            const int64_t pair = (s < ns && fl < nfh) ? (sub + s) * F + f0 + fl : 0;
            pk[u] = load_idx<IdxT>(a.idx, pair);
            pv[u] = a.x[pair];
        }
    };
    fetch_pairs(n_begin);

    // ---- stage tables, clear accumulators ---------------------------------
    for (int i = tid; i < FS; i += kBlock) s_nb[i] = i < nfh ? clamp_nbins(a.nbins[f0 + i], B) : 1;
    for (int i = tid; i < FS * KB; i += kBlock) {
        const int fl = i / KB;
        s_edge[i] = fl < nfh ? a.edges[static_cast<int64_t>(f0) * KB + i] : 0.0f;
    }
    for (int i = tid; i < FS * B; i += kBlock) {
        const int fl = i / B;
        s_iw[i] = fl < nfh ? a.iw[static_cast<int64_t>(f0) * B + i] : 0.0f;
    }
    for (int i = tid; i < FS * B * 2 * D; i += kBlock) s_hist[i] = 0.0f;
    for (int i = tid; i < FS * D; i += kBlock) s_db[i] = 0.0f;
    __syncthreads();
    for (int i = tid; i < FS * B * D; i += kBlock) {
        const int fl = i / (B * D);
        const int r = i - fl * (B * D);
        const int k = r / D;
        const int j = r - k * D;
        float w = 0.0f;
        if (fl < nfh) {
            const int n = s_nb[fl];
            if (k < n) w = quant<Q>(a.weight[(static_cast<int64_t>(f0 + fl) * B + phys_bin(k, n, B)) * D + j]);
        }
        s_qw[i] = w;
    }
    __syncthreads();

    const int lgw = LGW_T > 0 ? LGW_T : a.LGW;   // lanes per grad_output row (power of two)
    const int LG = kBlock / lgw;                  // lane groups (slices) per workgroup
    const int lg = tid / lgw;
    const int lc = tid - lg * lgw;
    const bool c_ok = lc < D / VEC;
    const int R = kP / LG;                        // sorted rows per slice
    const int NB = kP / kWave;                    // 64-pair blocks per sub-tile
    const int NBf = NT / kWave;                   // blocks per feature
    const int D2 = 2 * D, D3 = 3 * D;

    for (int64_t sub = n_begin; sub < n_end; sub += NT) {
        const int ns = static_cast<int>(min(static_cast<int64_t>(NT), n_end - sub));

        // A. pair info, stored feature-major (p = fl * NT + s)
#pragma unroll
        for (int u = 0; u < kPairsPerThread; ++u) {
            const int i = tid + u * kBlock;
            const int s = i / FS;
            const int fl = i - s * FS;
            int key = B;
            float qf = 0.0f;
            if (s < ns && fl < nfh) {
                const int k = clamp_bin(pk[u], s_nb[fl]);
                const float v = pv[u];
                const float e = s_edge[fl * KB + k];
                qf = quant<Q>((v - e) * s_iw[fl * B + k]);
                key = k | ((k > 0 && v == e) ? 0x8000 : 0);
            }
            s_info[fl * NT + s] = make_float2(qf, __int_as_float(key));
        }
        for (int i = tid; i < NB * KB; i += kBlock) s_cnt[i] = 0;
        __syncthreads();

        // B. rank of each pair among equal keys of its 64-pair block
        for (int b = wave; b < NB; b += kWavesPerBlock) {
            const int p = b * kWave + lane;
            const int k = __float_as_int(s_info[p].y) & 0x7fff;
            unsigned long long m = ~0ull;
            for (int bit = 0; bit < a.nbits; ++bit) {
                const bool set = (k >> bit) & 1;
                const unsigned long long bal = __ballot(set);
                m &= set ? bal : ~bal;
            }
            const unsigned long long lt = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
            const int rank = __popcll(m & lt);
            s_rank[p] = static_cast<uint8_t>(rank);
            if (rank == 0) s_cnt[b * KB + k] = static_cast<uint16_t>(__popcll(m));
        }
        __syncthreads();

        // C. per key: prefix over the feature's blocks; totals -> segment starts
        for (int kk = tid; kk < FS * KB; kk += kBlock) {
            const int fl = kk / KB;
            const int k = kk - fl * KB;
            int run = 0;
            for (int bb = 0; bb < NBf; ++bb) {
                const int ci = (fl * NBf + bb) * KB + k;
                const int cc = s_cnt[ci];
                s_cnt[ci] = static_cast<uint16_t>(run);
                run += cc;
            }
            s_seg[kk] = run;
        }
        __syncthreads();
        block_exclusive_scan(s_seg, FS * KB, s_tmp);

        // D. scatter: sorted position -> row descriptor {q(frac), key | edge | sample << 16}
        for (int p = tid; p < kP; p += kBlock) {
            const int fl = p / NT;
            const int s = p - fl * NT;
            const float2 inf = s_info[p];
            const int kb = __float_as_int(inf.y);
            const int k = kb & 0x7fff;
            const int slot = s_seg[fl * KB + k] + s_cnt[(p / kWave) * KB + k] + s_rank[p];
            s_sdesc[slot] = make_uint2(__float_as_uint(inf.x), static_cast<uint32_t>(kb & 0xffff) |
                                                                (static_cast<uint32_t>(s) << 16));
        }
        __syncthreads();

        // the next sub-tile's pair inputs travel while this one is reduced
        if (sub + NT < n_end) fetch_pairs(sub + NT);

        // F. slices of sorted rows, gradient rows prefetched a batch ahead
        {
            // Running sums of the slice's current key (feature, bin) -- packed as
            // fl << 16 | k -- and, with rounding quantisation, of its feature.
            // Padding rows (key B) and idle lanes (lc >= D / VEC) read a row of
            // zeros, so they add nothing and need no masking.
            int cur = -1, db_fl = -1;
            bool first_key = true, first_fl = true;
            float ab[VEC], aw[VEC], ad[VEC];
#pragma unroll
            for (int t = 0; t < VEC; ++t) ab[t] = aw[t] = ad[t] = 0.0f;
            if (lc == 0) {
                s_rkey[lg] = -1;
                s_rfl[lg] = -1;
            }
            float *rec = s_rec + lg * D3 + lc * VEC;

            // first key of the slice -> record; later keys -> straight into the
            // histogram (this slice is their only writer).  One read-modify-write
            // through a selected pointer keeps the code inlined per row small.
            auto flush_key = [&]() __attribute__((always_inline)) {
                if (cur < 0 || (cur & 0xffff) >= B) return;
                float *h = s_hist + (static_cast<size_t>(cur >> 16) * B + (cur & 0xffff)) * D2 + lc * VEC;
                float *dst = first_key ? rec : h;
                if (c_ok) {
                    float ob[VEC], ow[VEC];
                    lds_load_vec<VEC>(dst, ob);
                    lds_load_vec<VEC>(dst + D, ow);
#pragma unroll
                    for (int t = 0; t < VEC; ++t) {
                        ob[t] = first_key ? ab[t] : ob[t] + ab[t];
                        ow[t] = first_key ? aw[t] : ow[t] + aw[t];
                    }
                    lds_store_vec<VEC>(dst, ob);
                    lds_store_vec<VEC>(dst + D, ow);
                }
                if (first_key && lc == 0) s_rkey[lg] = cur;
                first_key = false;
            };
            auto flush_fl = [&]() __attribute__((always_inline)) {
                if (db_fl < 0) return;
                float *dst = first_fl ? rec + D2 : s_db + db_fl * D + lc * VEC;
                if (c_ok) {
                    float o[VEC];
                    lds_load_vec<VEC>(dst, o);
#pragma unroll
                    for (int t = 0; t < VEC; ++t) o[t] = first_fl ? ad[t] : o[t] + ad[t];
                    lds_store_vec<VEC>(dst, o);
                }
                if (first_fl && lc == 0) s_rfl[lg] = db_fl;
                first_fl = false;
            };

            // sorted position r -> feature r / NT (NT is a power of two)
            const int nt_shift = __ffs(NT) - 1;
            float gA[kUB][VEC], gB[kUB][VEC];

            // gradient rows of this sub-tile: 32-bit element offsets from the
            // sub-tile's first pair (the planner keeps NT * F * D below 2^31)
            const char *gsub = static_cast<const char *>(a.g) +
                               ((sub * F + f0) * D) * static_cast<int64_t>(GD == PLE_DTYPE_F32 ? 4 : 2);
            const int rowF = F * D;

            auto issue = [&](int rb, float (&gv)[kUB][VEC]) __attribute__((always_inline)) {
#pragma unroll
                for (int u = 0; u < kUB; ++u) {
                    const int r = rb + u;
                    const int fl = r >> nt_shift;
                    const uint32_t dw = s_sdesc[r].y;
                    const int s = static_cast<int>(dw >> 16);
                    // every lane loads, with no branch around the load (so the
                    // compiler waits for each batch separately); padding rows
                    // and idle lanes load zeros
                    const bool ok = c_ok && static_cast<int>(dw & 0x7fff) < B;
                    const void *src = ok ? static_cast<const void *>(gsub) : static_cast<const void *>(g_zero_row);
                    const int at = ok ? s * rowF + fl * D + lc * VEC : 0;
                    load_grad_vec<GD, VEC>(src, at, gv[u]);   // 16-bit zeros decode to +0 too
                }
            };

            // weight row and inverse width of the current key, reloaded from LDS
            // when the key changes (idle lanes read column 0; their g is 0)
            const int lcx = c_ok ? lc : 0;
            float wk[VEC];
            float iwk = 0.0f;
#pragma unroll
            for (int t = 0; t < VEC; ++t) wk[t] = 0.0f;
            auto process = [&](int rb, const float (&gv)[kUB][VEC]) __attribute__((always_inline)) {
                uint2 dsc[kUB];
#pragma unroll
                for (int u = 0; u < kUB; ++u) dsc[u] = s_sdesc[rb + u];
#pragma unroll
                for (int u = 0; u < kUB; ++u) {
                    const int r = rb + u;
                    const int fl = r >> nt_shift;
                    const float qf = __uint_as_float(dsc[u].x);
                    const uint32_t dw = dsc[u].y;
                    const int k = static_cast<int>(dw & 0x7fff);
                    const int s = static_cast<int>(dw >> 16);
                    const int key = (fl << 16) | k;
                    if (key != cur) {
                        flush_key();
#pragma unroll
                        for (int t = 0; t < VEC; ++t) ab[t] = aw[t] = 0.0f;
                        if constexpr (kRawDb) {
                            if (fl != db_fl) {
                                flush_fl();
#pragma unroll
                                for (int t = 0; t < VEC; ++t) ad[t] = 0.0f;
                                db_fl = fl;
                            }
                        }
                        cur = key;
                        const int kr = k < B ? k : 0;   // padding: any row (its g is 0)
                        lds_load_vec<VEC>(s_qw + (static_cast<size_t>(fl) * B + kr) * D + lcx * VEC, wk);
                        iwk = s_iw[fl * B + kr];
                    }
                    float gq[VEC];
                    float dot = 0.0f;
#pragma unroll
                    for (int t = 0; t < VEC; ++t) {
                        gq[t] = quant<Q>(gv[u][t]);
                        ab[t] += gq[t];
                        aw[t] = fmaf(qf, gq[t], aw[t]);
                        if constexpr (kRawDb) ad[t] += gv[u][t];
                        dot = fmaf(gq[t], wk[t], dot);
                    }
                    float part = dot * iwk;
                    if (dw & 0x8000) {                      // x on the bin's left edge (k >= 1)
                        float wp[VEC];
                        lds_load_vec<VEC>(s_qw + (static_cast<size_t>(fl) * B + k - 1) * D + lcx * VEC, wp);
                        float dot2 = 0.0f;
#pragma unroll
                        for (int t = 0; t < VEC; ++t) dot2 = fmaf(gq[t], wp[t], dot2);
                        part = fmaf(dot2, s_iw[fl * B + k - 1], part);
                    }
                    if constexpr (LGW_T > 0) part = group_sum<LGW_T>(part);
                    else part = group_sum_rt(part, lgw);
                    if (lc == 0) s_dx[(fl << nt_shift) + s] = part;
                }
            };

            // Two register buffers: batch b+1 is in flight while batch b is
            // reduced.  Every issue is unconditional (the one after the last
            // batch re-reads the slice's first rows and is discarded), so the
            // loop carries the same loads on every path and the waits stay
            // per batch.
            const int r0 = lg * R;
            const int r1 = r0 + R;
            if (R >= 2 * kUB) {
                issue(r0, gA);
                for (int rb = r0; rb < r1; rb += 2 * kUB) {
                    issue(rb + kUB, gB);
                    process(rb, gA);
                    issue(rb + 2 * kUB < r1 ? rb + 2 * kUB : r0, gA);
                    process(rb + kUB, gB);
                }
            } else {
                for (int rb = r0; rb < r1; rb += kUB) {
                    issue(rb, gA);
                    process(rb, gA);
                }
            }
            flush_key();
            if constexpr (kRawDb) flush_fl();
        }
        __syncthreads();

        // G. slice records, one run of equal keys (features) per head, in order
        if (c_ok) {
            const int key = s_rkey[lg];
            if (key >= 0 && (lg == 0 || s_rkey[lg - 1] != key)) {
                float sb[VEC], sw[VEC];
#pragma unroll
                for (int t = 0; t < VEC; ++t) sb[t] = sw[t] = 0.0f;
                for (int j = lg; j < LG && s_rkey[j] == key; ++j) {
                    const float *rj = s_rec + j * D3 + lc * VEC;
#pragma unroll
                    for (int t = 0; t < VEC; ++t) {
                        sb[t] += rj[t];
                        sw[t] += rj[D + t];
                    }
                }
                float *h = s_hist + (static_cast<size_t>(key >> 16) * B + (key & 0xffff)) * D2 + lc * VEC;
#pragma unroll
                for (int t = 0; t < VEC; ++t) {
                    h[t] += sb[t];
                    h[D + t] += sw[t];
                }
            }
            const int rfl = kRawDb ? s_rfl[lg] : -1;
            if (rfl >= 0 && (lg == 0 || s_rfl[lg - 1] != rfl)) {
                float sd[VEC];
#pragma unroll
                for (int t = 0; t < VEC; ++t) sd[t] = 0.0f;
                for (int j = lg; j < LG && s_rfl[j] == rfl; ++j) {
                    const float *rj = s_rec + j * D3 + D2 + lc * VEC;
#pragma unroll
                    for (int t = 0; t < VEC; ++t) sd[t] += rj[t];
                }
#pragma unroll
                for (int t = 0; t < VEC; ++t) s_db[rfl * D + lc * VEC + t] += sd[t];
            }
        }

        // H. dx, coalesced along the group's features
        if (a.dx) {
#pragma unroll
            for (int u = 0; u < kPairsPerThread; ++u) {
                const int i = tid + u * kBlock;
                const int s = i / FS;
                const int fl = i - s * FS;
                if (s < ns && fl < nfh) a.dx[(sub + s) * F + f0 + fl] = s_dx[fl * NT + s];
            }
        }
        __syncthreads();
    }

    // chunk partials
    if (a.part) {
        float *dst = a.part + (static_cast<int64_t>(c) * F + f0) * B * D2;
        for (int i = tid; i < FS * B * D2; i += kBlock) {
            const int fl = i / (B * D2);
            const int k = (i - fl * B * D2) / D2;
            if (fl < nfh && k < s_nb[fl]) dst[i] = s_hist[i];
        }
        if constexpr (kRawDb) {
            float *dstb = a.part_db + (static_cast<int64_t>(c) * F + f0) * D;
            for (int i = tid; i < FS * D; i += kBlock)
                if (i / D < nfh) dstb[i] = s_db[i];
        }
    }
}

// ---------------------------------------------------------------------------
// fallback kernels
// ---------------------------------------------------------------------------

// One 16-lane group per (sample, feature) pair.
template <int GD, int Q, typename IdxT>
__global__ __launch_bounds__(kBlock) void ple_bwd_simple_dx_kernel(BwdArgs a) {
    constexpr int kLanes = 16;
    const int64_t pairs = a.N * a.F;
    const int64_t grp = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) / kLanes;
    const int gl = threadIdx.x % kLanes;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * (kBlock / kLanes);
    const int B = a.B, D = a.D;
    for (int64_t p = grp; p < pairs; p += stride) {   // uniform per 16-lane group
        const int f = static_cast<int>(p % a.F);
        const int n = clamp_nbins(a.nbins[f], B);
        const int k = clamp_bin(load_idx<IdxT>(a.idx, p), n);
        const float *w = a.weight + (static_cast<int64_t>(f) * B + phys_bin(k, n, B)) * D;
        const float v = a.x[p];
        const bool edge = (k > 0) && (v == a.edges[static_cast<int64_t>(f) * (B + 1) + k]);
        const float *wp = a.weight + (static_cast<int64_t>(f) * B + (k > 0 ? k - 1 : 0)) * D;
        float s = 0.0f, s2 = 0.0f;
        for (int j = gl; j < D; j += kLanes) {
            const float gv = quant<Q>(load_grad<GD>(a.g, p * D + j));
            s = fmaf(gv, quant<Q>(w[j]), s);
            if (edge) s2 = fmaf(gv, quant<Q>(wp[j]), s2);
        }
#pragma unroll
        for (int off = kLanes / 2; off > 0; off >>= 1) {
            s += __shfl_xor(s, off, kLanes);
            s2 += __shfl_xor(s2, off, kLanes);
        }
        if (gl == 0) {
            float r = s * a.iw[static_cast<int64_t>(f) * B + k];
            if (edge) r = fmaf(s2, a.iw[static_cast<int64_t>(f) * B + k - 1], r);
            a.dx[p] = r;
        }
    }
}

// One wave per (feature, sample chunk); lane j owns column j (D <= 64) and
// walks the chunk in sample order, folding runs of equal bins into its own
// LDS cells.
template <int GD, int Q, typename IdxT>
__global__ __launch_bounds__(kWave) void ple_bwd_simple_hist_kernel(BwdArgs a) {
    extern __shared__ float smem[];
    const int B = a.B, D = a.D, F = a.F;
    float *hb = smem;
    float *hw = smem + B * D;
    const int f = blockIdx.x % F;
    const int c = blockIdx.x / F;
    const int j = threadIdx.x;
    const bool jok = j < D;
    const int n_real = clamp_nbins(a.nbins[f], B);
    for (int i = j; i < n_real * D; i += kWave) {
        hb[i] = 0.0f;
        hw[i] = 0.0f;
    }
    __syncthreads();
    const int64_t n_begin = static_cast<int64_t>(c) * a.NC;
    const int64_t n_end = min(a.N, n_begin + a.NC);
    const float *e = a.edges + static_cast<int64_t>(f) * (B + 1);
    const float *iwr = a.iw + static_cast<int64_t>(f) * B;
    int kc = -1;
    float cb = 0.0f, cw = 0.0f, cdb = 0.0f;
    constexpr int kBatch = 16;
    for (int64_t n0 = n_begin; n0 < n_end; n0 += kBatch) {
        int kk[kBatch];
        float xv[kBatch];
        float gv[kBatch];
#pragma unroll
        for (int t = 0; t < kBatch; ++t) {
            const int64_t n = n0 + t;
            const bool ok = n < n_end;
            const int64_t p = n * F + f;
            kk[t] = ok ? clamp_bin(load_idx<IdxT>(a.idx, p), n_real) : 0;
            xv[t] = ok ? a.x[p] : 0.0f;
            gv[t] = (ok && jok) ? load_grad<GD>(a.g, p * D + j) : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < kBatch; ++t) {
            if (n0 + t >= n_end) break;
            const int k = kk[t];
            const float qf = quant<Q>((xv[t] - e[k]) * iwr[k]);
            const float graw = gv[t];
            const float gq = quant<Q>(graw);
            if (k != kc) {
                if (kc >= 0 && jok) {
                    hb[kc * D + j] += cb;
                    hw[kc * D + j] += cw;
                }
                kc = k;
                cb = gq;
                cw = qf * gq;
            } else {
                cb += gq;
                cw = fmaf(qf, gq, cw);
            }
            cdb += graw;
        }
    }
    if (kc >= 0 && jok) {
        hb[kc * D + j] += cb;
        hw[kc * D + j] += cw;
    }
    __syncthreads();
    float *dst = a.part + (static_cast<int64_t>(c) * F + f) * B * 2 * D;
    for (int i = j; i < n_real * D; i += kWave) {
        const int k = i / D;
        const int jj = i - k * D;
        dst[k * 2 * D + jj] = hb[i];
        dst[k * 2 * D + D + jj] = hw[i];
    }
    if (jok) a.part_db[(static_cast<int64_t>(c) * F + f) * D + j] = cdb;
}

// ---------------------------------------------------------------------------
// finalize: one workgroup per feature
// ---------------------------------------------------------------------------

// Sums the chunk partials of every (bin, column) in chunk order into LDS,
// then one lane per column takes the suffix over logical bins:
// dW[phys(k)] = weighted[k] + sum_{m>k} bucket[m]; slots no bin maps to get
// 0.  The bias gradient sums its chunk partials in chunk order.
__global__ __launch_bounds__(kBlock) void ple_bwd_finalize_kernel(BwdArgs a) {
    extern __shared__ float tot[];       // [n][2D]
    const int f = blockIdx.x;
    const int B = a.B, D = a.D, F = a.F;
    const int D2 = 2 * D;
    const int n = clamp_nbins(a.nbins[f], B);
    const int tid = threadIdx.x;
    const int64_t cstride = static_cast<int64_t>(F) * B * D2;
    const float *src = a.part + static_cast<int64_t>(f) * B * D2;
    const bool need_tot = a.dw || (a.db && a.db_from_buckets);
    if (need_tot) {
        for (int i = tid; i < n * D2; i += kBlock) {
            float s = 0.0f;
#pragma unroll 8
            for (int cc = 0; cc < a.Cd; ++cc) s += src[cc * cstride + i];
            tot[i] = s;
        }
        __syncthreads();
    }
    if (a.dw) {
        for (int j = tid; j < D; j += kBlock) {
            float fut = 0.0f;
            for (int k = n - 1; k >= 0; --k) {
                a.dw[(static_cast<int64_t>(f) * B + phys_bin(k, n, B)) * D + j] = tot[k * D2 + D + j] + fut;
                fut += tot[k * D2 + j];
            }
        }
        for (int i = tid; i < (B - n) * D; i += kBlock)
            a.dw[(static_cast<int64_t>(f) * B + (n - 1) + i / D) * D + i % D] = 0.0f;
    }
    if (a.db) {
        for (int j = tid; j < D; j += kBlock) {
            float s = 0.0f;
            if (a.db_from_buckets) {
                for (int k = n - 1; k >= 0; --k) s += tot[k * D2 + j];
            } else {
                for (int cc = 0; cc < a.Cd; ++cc) s += a.part_db[(static_cast<int64_t>(cc) * F + f) * D + j];
            }
            a.db[static_cast<int64_t>(f) * D + j] = s;
        }
    }
}

// ---------------------------------------------------------------------------
// planning
// ---------------------------------------------------------------------------

constexpr size_t kPartialBudget = 64ull << 20;   // bytes of chunk partials
constexpr size_t kFusedLdsTwoPerCu = 80 * 1024;

int env_int(const char *name, int dflt) {
    const char *s = getenv(name);
    if (!s || !*s) return dflt;
    return atoi(s);
}

struct BwdPlan {
    bool fused;
    int vec;
    int C, Cd;
    int64_t NC;
    size_t lds;
    size_t part_bytes, part_db_bytes;
    BwdArgs geo;     // fused geometry and LDS offsets
    size_t total() const { return align_up(part_bytes, 256) + align_up(part_db_bytes, 256); }
};

size_t fused_layout(BwdArgs &g, int FS, int P, int B, int D, int LG) {
    size_t off = 0;
    auto take = [&](int &field, size_t bytes) {
        field = static_cast<int>(off);
        off = align_up(off + bytes, 16);
    };
    const size_t KB = static_cast<size_t>(B) + 1;
    take(g.o_qw, 4ull * FS * B * D);
    take(g.o_hist, 8ull * FS * B * D);
    take(g.o_db, 4ull * FS * D);
    take(g.o_edge, 4ull * FS * KB);
    take(g.o_iw, 4ull * FS * B);
    take(g.o_nb, 4ull * FS);
    take(g.o_info, 8ull * P);
    take(g.o_order, 8ull * P);
    take(g.o_rank, 1ull * P);
    take(g.o_cnt, 2ull * (P / kWave) * KB);
    take(g.o_seg, 4ull * (FS * KB + 1));
    take(g.o_dx, 4ull * P);
    take(g.o_rec, 12ull * LG * D);
    take(g.o_rkey, 4ull * LG);
    take(g.o_rfl, 4ull * LG);
    take(g.o_tmp, 4ull * kWavesPerBlock);
    return off;
}

// g_align16: the gradient's base address is 16-byte aligned
BwdPlan plan_backward(int64_t N, int64_t F, int64_t B, int64_t D, bool g_align16) {
    BwdPlan pl{};
    const int cus = device_cu_count();
    pl.fused = false;
    // fused geometry: VEC=4 rows of D/4 lanes when D allows, else one column
    // per lane; lane groups of a power-of-two width between 2 and 64
    if (B <= 4096 && static_cast<int64_t>(kP) * F * D < INT32_MAX && env_int("PLE_BWD_SIMPLE", 0) == 0) {
        // 8 floats per lane when D allows (half the lanes, and half the per-row
        // overhead, of 4 per lane)
        const int vec = !g_align16 ? 1 : (D % 8 == 0 ? 8 : (D % 4 == 0 && D >= 8 ? 4 : 1));
        const int uv = static_cast<int>(D / vec);
        int lgw = 2;
        while (lgw < uv) lgw *= 2;
        if (lgw <= kWave) {
            const int LG = kBlock / lgw;
            int best_fs = 0;
            size_t best_lds = 0;
            BwdArgs geo{};
            for (int fs = 4; fs >= 1; fs /= 2) {
                if (fs > 1 && fs > F) continue;
                BwdArgs t{};
                const size_t lds = fused_layout(t, fs, kP, static_cast<int>(B), static_cast<int>(D), LG);
                if (lds <= kFusedLdsTwoPerCu || (fs == 1 && lds <= kLdsMax)) {
                    best_fs = fs;
                    best_lds = lds;
                    geo = t;
                    break;
                }
            }
            const int fs_env = env_int("PLE_BWD_FS", 0);
            if (fs_env == 1 || fs_env == 2 || fs_env == 4 || fs_env == 8 || fs_env == 16) {
                BwdArgs t{};
                const size_t lds = fused_layout(t, fs_env, kP, static_cast<int>(B), static_cast<int>(D), LG);
                if (lds <= kLdsMax) {
                    best_fs = fs_env;
                    best_lds = lds;
                    geo = t;
                }
            }
            if (best_fs > 0) {
                pl.fused = true;
                pl.vec = vec;
                pl.lds = best_lds;
                geo.FS = best_fs;
                geo.G = static_cast<int>((F + best_fs - 1) / best_fs);
                geo.P = kP;
                geo.NT = kP / best_fs;
                geo.LGW = lgw;
                int nbits = 0;
                while ((1ll << nbits) <= B) ++nbits;      // keys 0..B
                geo.nbits = nbits;
                pl.geo = geo;
                const int64_t per_chunk = F * B * 2 * D * 4;
                int64_t c = (static_cast<int64_t>(env_int("PLE_BWD_WG_PER_CU", 4)) * cus + geo.G - 1) / geo.G;
                const int64_t budget_c = static_cast<int64_t>(kPartialBudget) / per_chunk;
                if (c > budget_c) c = budget_c;
                const int64_t max_c = (N + geo.NT - 1) / geo.NT;   // at least one sub-tile per chunk
                if (c > max_c) c = max_c;
                if (c < 1) c = 1;
                int64_t nc = (N + c - 1) / c;
                nc = (nc + geo.NT - 1) / geo.NT * geo.NT;
                pl.NC = nc;
                pl.Cd = static_cast<int>((N + nc - 1) / nc);
                pl.C = (pl.Cd + kNumXcd - 1) / kNumXcd * kNumXcd;
            }
        }
    }
    if (!pl.fused) {
        const int64_t waves = 32 * static_cast<int64_t>(cus);
        int64_t c = (waves + F - 1) / F;
        const int64_t per_chunk = F * B * 2 * D * 4;
        const int64_t budget_c = static_cast<int64_t>(kPartialBudget) / (per_chunk > 0 ? per_chunk : 1);
        if (c > budget_c) c = budget_c;
        if (c > 1024) c = 1024;
        const int64_t max_c = (N + 63) / 64;
        if (c > max_c) c = max_c;
        if (c < 1) c = 1;
        pl.NC = (N + c - 1) / c;
        pl.C = pl.Cd = static_cast<int>((N + pl.NC - 1) / pl.NC);
        pl.lds = static_cast<size_t>(B) * D * 2 * sizeof(float);
    }
    pl.part_bytes = static_cast<size_t>(pl.Cd) * F * B * 2 * D * sizeof(float);
    pl.part_db_bytes = static_cast<size_t>(pl.Cd) * F * D * sizeof(float);
    return pl;
}

// Bin indices are uint8 (up to 256 bins) or int16 (up to 32766 bins, the
// largest key the fused sort encodes).
template <int GD, int Q, int VEC, int LGW>
hipError_t launch_fused_idx(const BwdArgs &a, int idxb, dim3 grid, size_t lds, hipStream_t s) {
    if (idxb == 1) hipLaunchKernelGGL((ple_bwd_fused_kernel<GD, Q, VEC, LGW, uint8_t>), grid, dim3(kBlock), lds, s, a);
    else hipLaunchKernelGGL((ple_bwd_fused_kernel<GD, Q, VEC, LGW, int16_t>), grid, dim3(kBlock), lds, s, a);
    return hipGetLastError();
}

// Lane-group width as a template argument for the VEC=4 rows (DPP
// reductions); the one-column-per-lane variant takes it at run time.
template <int GD, int Q>
hipError_t launch_fused(const BwdArgs &a, int vec, int idxb, dim3 grid, size_t lds, hipStream_t s) {
    if (vec == 8) {
        switch (a.LGW) {
            case 2: return launch_fused_idx<GD, Q, 8, 2>(a, idxb, grid, lds, s);
            case 4: return launch_fused_idx<GD, Q, 8, 4>(a, idxb, grid, lds, s);
            default: return launch_fused_idx<GD, Q, 8, 8>(a, idxb, grid, lds, s);
        }
    }
    if (vec == 4) {
        switch (a.LGW) {
            case 4: return launch_fused_idx<GD, Q, 4, 4>(a, idxb, grid, lds, s);
            case 8: return launch_fused_idx<GD, Q, 4, 8>(a, idxb, grid, lds, s);
            default: return launch_fused_idx<GD, Q, 4, 16>(a, idxb, grid, lds, s);
        }
    }
    return launch_fused_idx<GD, Q, 1, 0>(a, idxb, grid, lds, s);
}

template <int GD, int Q>
hipError_t launch_typed(BwdArgs a, const BwdPlan &pl, int idxb, bool want_dx, bool want_dwdb, hipStream_t s) {
    hipError_t e = hipSuccess;
    if (pl.fused) {
        a.db_from_buckets = Q == PLE_DTYPE_F32;
        const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.G) * pl.C));
        e = launch_fused<GD, Q>(a, pl.vec, idxb, grid, pl.lds, s);
        if (e != hipSuccess) return e;
    } else {
        if (want_dx) {
            const int64_t pairs = a.N * a.F;
            int64_t blocks = (pairs + (kBlock / 16) - 1) / (kBlock / 16);
            const int64_t cap = static_cast<int64_t>(device_cu_count()) * 16;
            if (blocks > cap) blocks = cap;
            if (blocks < 1) blocks = 1;
            if (idxb == 1) hipLaunchKernelGGL((ple_bwd_simple_dx_kernel<GD, Q, uint8_t>), dim3(blocks), dim3(kBlock), 0, s, a);
            else hipLaunchKernelGGL((ple_bwd_simple_dx_kernel<GD, Q, int16_t>), dim3(blocks), dim3(kBlock), 0, s, a);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        if (want_dwdb) {
            const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.F) * pl.C));
            if (idxb == 1) hipLaunchKernelGGL((ple_bwd_simple_hist_kernel<GD, Q, uint8_t>), grid, dim3(kWave), pl.lds, s, a);
            else hipLaunchKernelGGL((ple_bwd_simple_hist_kernel<GD, Q, int16_t>), grid, dim3(kWave), pl.lds, s, a);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
    }
    if (want_dwdb) {
        const size_t lds = static_cast<size_t>(a.B) * 2 * a.D * sizeof(float);
        hipLaunchKernelGGL(ple_bwd_finalize_kernel, dim3(a.F), dim3(kBlock), lds, s, a);
        e = hipGetLastError();
    }
    return e;
}

// Supported (grad, quant) pairs: quant == grad (the reference operator, whose
// gradient arrives in the forward's output dtype) or an fp32 gradient with
// any quant (the fused-bias operator under autocast).
template <int GD>
hipError_t launch_q(const BwdArgs &a, const BwdPlan &pl, int q, int idxb, bool want_dx, bool want_dwdb, hipStream_t s) {
    if constexpr (GD == PLE_DTYPE_F32) {
        switch (q) {
            case PLE_DTYPE_F32: return launch_typed<GD, PLE_DTYPE_F32>(a, pl, idxb, want_dx, want_dwdb, s);
            case PLE_DTYPE_F16: return launch_typed<GD, PLE_DTYPE_F16>(a, pl, idxb, want_dx, want_dwdb, s);
            default: return launch_typed<GD, PLE_DTYPE_BF16>(a, pl, idxb, want_dx, want_dwdb, s);
        }
    } else {
        return launch_typed<GD, GD>(a, pl, idxb, want_dx, want_dwdb, s);
    }
}

}  // namespace

size_t backward_workspace_bytes(int64_t N, int64_t F, int64_t B, int64_t D) {
    // the plan depends on the gradient's alignment; report the largest need
    const size_t a = plan_backward(N, F, B, D, true).total();
    const size_t b = plan_backward(N, F, B, D, false).total();
    return a > b ? a : b;
}

int backward_run(const BackwardRequest &r) {
    const bool want_dx = r.dx != nullptr;
    const bool want_dwdb = r.dw != nullptr || r.db != nullptr;
    if (r.grad_dtype != PLE_DTYPE_F32 && r.quant != r.grad_dtype) return PLE_E_UNSUPPORTED;
    const uintptr_t gaddr = reinterpret_cast<uintptr_t>(r.g);
    const int gbytes = r.grad_dtype == PLE_DTYPE_F32 ? 4 : 2;
    if (gaddr % gbytes != 0) return PLE_E_MISALIGNED;
    BwdPlan pl = plan_backward(r.N, r.F, r.B, r.D, gaddr % 16 == 0);
    if (!pl.fused && want_dwdb && pl.lds > kLdsMax) return PLE_E_UNSUPPORTED;
    const size_t need = pl.total();
    if (want_dwdb && (r.workspace == nullptr || r.workspace_bytes < need ||
                      reinterpret_cast<uintptr_t>(r.workspace) % 256 != 0))
        return PLE_E_WORKSPACE;
    if (static_cast<int64_t>(pl.fused ? pl.geo.G : r.F) * pl.C > INT32_MAX) return PLE_E_TOO_LARGE;
    BwdArgs a = pl.geo;
    a.g = r.g; a.x = r.x; a.edges = r.edges; a.iw = r.iw; a.nbins = r.nbins; a.weight = r.weight;
    a.idx = r.idx; a.dx = r.dx; a.dw = r.dw; a.db = r.db;
    char *ws = static_cast<char *>(r.workspace);
    a.part = want_dwdb ? reinterpret_cast<float *>(ws) : nullptr;
    a.part_db = want_dwdb ? reinterpret_cast<float *>(ws + align_up(pl.part_bytes, 256)) : nullptr;
    a.N = r.N; a.F = static_cast<int>(r.F); a.B = static_cast<int>(r.B); a.D = static_cast<int>(r.D);
    a.C = pl.C; a.Cd = pl.Cd; a.NC = pl.NC;
    const int idxb = idx_bytes_for(r.B);
    hipError_t e;
    switch (r.grad_dtype) {
        case PLE_DTYPE_F32: e = launch_q<PLE_DTYPE_F32>(a, pl, r.quant, idxb, want_dx, want_dwdb, r.stream); break;
        case PLE_DTYPE_F16: e = launch_q<PLE_DTYPE_F16>(a, pl, r.quant, idxb, want_dx, want_dwdb, r.stream); break;
        default: e = launch_q<PLE_DTYPE_BF16>(a, pl, r.quant, idxb, want_dx, want_dwdb, r.stream); break;
    }
    return e == hipSuccess ? PLE_OK : static_cast<int>(e);
}

}  // namespace ple
