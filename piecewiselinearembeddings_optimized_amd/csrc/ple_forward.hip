// Forward kernel of the fused PLE path (gfx950).
//
// One workgroup owns a group of FS features and a chunk of samples.  It
// stages, per feature, the bin edges, the inverse widths and a [bins x 2D]
// table {prefix of quantised weights | quantised weight row} in LDS, then its
// four waves stream wave tiles of 64 (sample, feature) pairs: each lane
// bin-searches one pair in LDS, the pair's (bin, fraction) reaches the lanes
// that store that pair's D outputs through ds_bpermute, and the outputs leave
// as 16-byte stores covering whole sample rows of the group.
//
// Arithmetic per output element is the reference's (forward_cuda.cu:135-178,
// 208-283): prefix accumulated in fp32 in bin order, then
// fma(q(frac), q(W[phys(k)]), prefix[k]), rounded to the output dtype.
//
// Epilogues (the module's elementwise tail, reference module.py:230-248,
// fused into the store; the output is then fp32):
//   bias       v = x_ple + bias                      (version A)
//   bias_relu  v = relu(x_ple + bias)
//   lin        v = (lin_b + lin_w * x) + x_ple        (version B, linear0)
//   lin_relu   v = (lin_b + lin_w * x) + relu(x_ple)
// With ReLU the store also writes one bit per element, set where the ReLU
// passes its input (input > 0, or NaN), for the backward.
//
// Tables too large for LDS (many bins times a wide row) take
// ple_fwd_wide_kernel: LDS holds checkpoints of the prefix every S bins, and
// each output continues the fold from its checkpoint with weights read from
// global memory -- the same fp32 additions in the same order, so the same
// bits (the role of the reference's generic kernel, forward_cuda.cu:293-425,
// chosen at :478-512).

#include "ple_device.h"
#include "ple_internal.h"

namespace ple {
namespace {

struct FwdArgs {
    const float *x;
    const float *edges;
    const float *iw;
    const int32_t *nbins;
    const float *weight;
    const float *bias;
    const float *lin_w;     // [F, D] linear0 weight (version B) or NULL
    const float *lin_b;     // [F, D] linear0 bias
    uint32_t *mask;         // [N, F, MW] ReLU pass bits, or NULL
    int MW;                 // mask words per (sample, feature) row = ceil(D / 32)
    void *out;
    void *idx;
    int64_t N;
    int F, B, D;
    int FS;       // features per workgroup (power of two, FS * DC/VEC <= 64)
    int G;        // workgroup columns = ceil(F / FS) feature groups x NCC column chunks
    int DC;       // columns per chunk (= D unless a row is wider than a wave's lanes)
    int NCC;      // column chunks per row (FS = 1 when NCC > 1)
    int C;        // sample chunks
    int64_t NC;   // samples per chunk
    int FB;       // threads per workgroup (kBlock or 2 * kBlock)
    int out_nt;   // table kernel: output stores with the non-temporal hint (see forward_run)
    // wide-table kernel: checkpoint stride (bins), LDS offsets (floats) of
    // the weight stage and of the edge / inverse-width tables, and whether
    // the edges and inverse widths are staged in LDS (else every ES-th edge
    // is, for the first steps of the bin search, and the rest is read from
    // global memory)
    int S, stage_off, edge_off, edges_lds, ES;
};

size_t fwd_lds_bytes(int64_t FS, int64_t B, int64_t D) {
    return 4 * (static_cast<size_t>(FS) * B * 2 * D   // table {prefix | weight}
                + static_cast<size_t>(FS) * (B + 1)   // edges
                + static_cast<size_t>(FS) * B         // inverse widths
                + static_cast<size_t>(FS));           // n_bins
}

constexpr int kStoreUnroll = 4;

enum : int { kEpiNone = 0, kEpiBias = 1, kEpiBiasRelu = 2, kEpiLin = 3, kEpiLinRelu = 4 };

// OR of v over the U consecutive lanes of a row (first lane: lane - u); every
// lane of the row receives it.  Power-of-two rows are aligned to U lanes.
__device__ __forceinline__ uint32_t row_or(uint32_t v, int U, int lane, int u) {
    if ((U & (U - 1)) == 0) {
        for (int off = 1; off < U; off <<= 1) v |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off));
        return v;
    }
    uint32_t acc = 0;
    for (int j = 0; j < U; ++j) acc |= static_cast<uint32_t>(__shfl(static_cast<int>(v), lane - u + j));
    return acc;
}

// One lane's VEC results of an output row (fp32 fma of prefix and fraction
// times weight) rounded through Q, the epilogue applied, stored as OUT at
// element `oi` of the output.  With ReLU the pass bits of the row's U lanes
// (this one is lane o_u of them) are gathered into the row's mask words at
// `mi`.  bvec / lwv: the lane's bias or linear0 weight (linear0 bias in bvec);
// xs: the sample's x (linear0).
template <int Q, int OUT, int EPI, int VEC, bool NT = true>
__device__ __forceinline__ void emit_segment(const FwdArgs &a, float (&r)[VEC], const float (&bvec)[VEC],
                                             const float (&lwv)[VEC], float xs, bool row_ok, int64_t oi,
                                             int64_t mi, int U, int lane, int o_u, int m_shift, int m_word) {
    constexpr bool HAS_BIAS = EPI == kEpiBias || EPI == kEpiBiasRelu;
    constexpr bool RELU = EPI == kEpiBiasRelu || EPI == kEpiLinRelu;
    constexpr bool LIN = EPI == kEpiLin || EPI == kEpiLinRelu;
    uint32_t mbits = 0;
#pragma unroll
    for (int t2 = 0; t2 < VEC; ++t2) {
        // (with no epilogue the output dtype is Q, and the store's own
        // rounding is this one)
        float o = EPI == kEpiNone ? r[t2] : quant<Q>(r[t2]);
        if constexpr (HAS_BIAS) o = o + bvec[t2];
        if constexpr (RELU) {
            // torch.relu: NaN passes, x <= 0 gives 0
            const bool pass = !(o <= 0.0f);
            mbits |= static_cast<uint32_t>(pass) << t2;
            o = pass ? o : 0.0f;
        }
        if constexpr (LIN) o = fmaf(lwv[t2], xs, bvec[t2]) + o;
        r[t2] = o;
    }
    if (row_ok) store_out<OUT, VEC, NT>(a.out, oi, r);
    if constexpr (RELU) {
        if (a.mask) {
            const uint32_t w0 = row_or(m_word == 0 ? mbits << m_shift : 0u, U, lane, o_u);
            const uint32_t w1 = a.MW > 1 ? row_or(m_word == 1 ? mbits << m_shift : 0u, U, lane, o_u) : 0u;
            if (row_ok && o_u == 0) {
                uint32_t *mp = a.mask + mi;
                mp[0] = w0;
                if (a.MW > 1) mp[1] = w1;
            }
        }
    }
}

// FB: threads per workgroup (256, or 512 where the tables leave room for at
// most two workgroups per CU: twice the waves per staged table); NT: output
// stores with the non-temporal hint where store_out gives them one
template <int Q, int OUT, int EPI, int VEC, typename IdxT, int FB, bool NT = true>
__global__ __launch_bounds__(FB) void ple_fwd_kernel(FwdArgs a) {
    constexpr int kWaves = FB / kWave;
    // wave tiles whose x is loaded during the table staging: with 512
    // threads (short output rows) 16 for 16-bit outputs (all of a wave's
    // tiles in the usual plans), 8 for fp32 ones, whose tiles' stores take
    // twice as long (fwd+bwd step: c3 136 -> 130 us with 8, c4 116 -> 123 us)
    constexpr int kXEarly = FB == 512 ? (OUT == PLE_DTYPE_F32 ? 8 : 16) : 1;
    constexpr bool HAS_BIAS = EPI == kEpiBias || EPI == kEpiBiasRelu;
    constexpr bool LIN = EPI == kEpiLin || EPI == kEpiLinRelu;
    extern __shared__ float smem[];
    const int FS = a.FS, B = a.B, D = a.D, F = a.F;

    int g, c;
    if (!decode_tile(blockIdx.x, a.G, a.C, g, c)) return;
    // A row wider than a wave's lanes is cut into column chunks, one per
    // workgroup (one feature a group then): columns c0 .. c0 + Dw - 1 of
    // the feature's table and output.
    const int cc = g % a.NCC;
    g /= a.NCC;
    const int c0 = cc * a.DC;
    const int Dw = min(a.DC, D - c0);
    const int rs = 2 * Dw;                                  // table row stride
    float *tbl = smem;
    float *sedge = tbl + static_cast<size_t>(FS) * B * 2 * a.DC;
    float *siw = sedge + FS * (B + 1);
    int *snb = reinterpret_cast<int *>(siw + FS * B);
    const int f0 = g * FS;
    const int nfh = min(FS, F - f0);
    const int64_t n_begin = static_cast<int64_t>(c) * a.NC;
    const int64_t n_end = min(a.N, n_begin + a.NC);
    if (n_begin >= n_end) return;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int SW = kWave / FS;      // samples per wave tile
    const int64_t n_tiles = (n_end - n_begin + SW - 1) / SW;
    // pair phase: lane -> (sample p_s, feature p_fl)
    const int p_s = lane / FS;
    const int p_fl = lane - p_s * FS;
    const bool p_fok = p_fl < nfh;
    // x of wave tile t (an out-of-range lane reads x[0] and ignores it, so
    // the load has no branch around it)
    auto load_x = [&](int64_t t) __attribute__((always_inline)) -> float {
        const int64_t pn = n_begin + t * SW + p_s;
        const bool ok = p_fok && (t < n_tiles) && (pn < n_end);
        return a.x[ok ? pn * F + f0 + p_fl : 0];
    };

    // ---- stage the per-feature tables ------------------------------------
    for (int i = tid; i < FS; i += FB) snb[i] = i < nfh ? clamp_nbins(a.nbins[f0 + i], B) : 1;
    for (int i = tid; i < FS * (B + 1); i += FB) {
        const int fl = i / (B + 1);
        sedge[i] = fl < nfh ? a.edges[static_cast<int64_t>(f0) * (B + 1) + i] : 0.0f;
    }
    for (int i = tid; i < FS * B; i += FB) {
        const int fl = i / B;
        siw[i] = fl < nfh ? a.iw[static_cast<int64_t>(f0) * B + i] : 0.0f;
    }
    __syncthreads();

    const int U = Dw / VEC;
    for (int i = tid; i < FS * B * U; i += FB) {
        const int fl = i / (B * U);
        const int r = i - fl * (B * U);
        const int k = r / U;
        const int u = r - k * U;
        if (fl < nfh) {
            const int n = snb[fl];
            if (k < n) {
                const int p = phys_bin(k, n, B);
                const float *src = a.weight + ((static_cast<int64_t>(f0 + fl) * B + p) * D + c0 + u * VEC);
                float *dst = tbl + (static_cast<size_t>(fl) * B + k) * rs + Dw + u * VEC;
                if constexpr (VEC % 4 == 0) {
#pragma unroll
                    for (int h = 0; h < VEC; h += 4) {
                        const float4 w = *reinterpret_cast<const float4 *>(src + h);
                        dst[h] = quant<Q>(w.x);
                        dst[h + 1] = quant<Q>(w.y);
                        dst[h + 2] = quant<Q>(w.z);
                        dst[h + 3] = quant<Q>(w.w);
                    }
                } else {
#pragma unroll
                    for (int h = 0; h < VEC; ++h) dst[h] = quant<Q>(src[h]);
                }
            }
        }
    }
    // x of the wave's first kXEarly tiles, loaded while the tables are
    // staged: after a kernel that streamed other data through the caches, x
    // comes from memory, and with short rows (16-bit or narrow outputs, 512
    // threads) a tile's stores take less time than that load
    float x_early[kXEarly];
#pragma unroll
    for (int i = 0; i < kXEarly; ++i) x_early[i] = load_x(wave + static_cast<int64_t>(i) * kWaves);
    __syncthreads();

    // prefix over logical bins, one lane per (feature, column), in bin order
    for (int col = tid; col < FS * Dw; col += FB) {
        const int fl = col / Dw;
        const int j = col - fl * Dw;
        if (fl < nfh) {
            const int n = snb[fl];
            float *base = tbl + static_cast<size_t>(fl) * B * rs;
            float acc = 0.0f;
            int k = 0;
            for (; k + 8 <= n; k += 8) {
                float w[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) w[t] = base[(k + t) * rs + Dw + j];
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    base[(k + t) * rs + j] = acc;
                    acc += w[t];
                }
            }
            for (; k < n; ++k) {
                const float w = base[k * rs + Dw + j];
                base[k * rs + j] = acc;
                acc += w;
            }
        }
    }
    __syncthreads();

    // ---- stream wave tiles -------------------------------------------------
    const int Lv = FS * U;          // vector slots per sample row of the group
    const int R = kWave / Lv;       // sample rows per store instruction

    const float *e_row = sedge + p_fl * (B + 1);
    const float *iw_row = siw + p_fl * B;
    const int p_n = snb[p_fl];

    // store phase: lane -> (row o_s, feature o_fl, vector o_u), fixed per lane
    const int o_s = lane / Lv;
    const int o_v = lane - o_s * Lv;
    const int o_fl = o_v / U;
    const int o_u = o_v - o_fl * U;
    const bool o_ok = (o_s < R) && (o_fl < nfh);
    // per-lane epilogue parameters: bias, or linear0's weight and bias
    float bvec[VEC], lwv[VEC];
#pragma unroll
    for (int t = 0; t < VEC; ++t) bvec[t] = lwv[t] = 0.0f;
    if constexpr (HAS_BIAS || LIN) {
        if (o_ok) {
            const int64_t pofs = static_cast<int64_t>(f0 + o_fl) * D + c0 + o_u * VEC;
#pragma unroll
            for (int t = 0; t < VEC; ++t) {
                bvec[t] = HAS_BIAS ? a.bias[pofs + t] : a.lin_b[pofs + t];
                if constexpr (LIN) lwv[t] = a.lin_w[pofs + t];
            }
        }
    }
    // ReLU bits: element j of a row is bit j % 32 of word j / 32 (a lane's
    // VEC elements never straddle a word: VEC divides 32; the epilogues run
    // rows of one chunk)
    const int m_shift = (o_u * VEC) & 31;
    const int m_word = (o_u * VEC) >> 5;
    const float *o_tbl = tbl + static_cast<size_t>(o_fl) * B * rs + o_u * VEC;

    const int64_t row_elems = static_cast<int64_t>(F) * D;

    // one wave tile: bin search, bin index, and the tile's output rows
    auto tile = [&](int64_t t, float xv) __attribute__((always_inline)) {
        const int64_t n0 = n_begin + t * SW;
        const int64_t pn = n0 + p_s;
        const bool pvalid = p_fok && (pn < n_end);
        const int64_t pidx = pn * F + f0 + p_fl;
        const float v = pvalid ? xv : 0.0f;
        const int k = find_bin(v, e_row, p_n);
        const float frac = (v - e_row[k]) * iw_row[k];
        const float qf = quant<Q>(frac);
        if (pvalid && cc == 0) static_cast<IdxT *>(a.idx)[pidx] = static_cast<IdxT>(k);

        // kStoreUnroll store instructions per step: their shuffles and table
        // reads are issued together, then the stores
        for (int sb = 0; sb < SW; sb += R * kStoreUnroll) {
            int ks[kStoreUnroll];
            float qs[kStoreUnroll], xs[kStoreUnroll];
#pragma unroll
            for (int q = 0; q < kStoreUnroll; ++q) {
                const int src = ((sb + q * R + o_s) * FS + o_fl) & (kWave - 1);
                ks[q] = __shfl(k, src);
                qs[q] = __shfl(qf, src);
                if constexpr (LIN) xs[q] = __shfl(v, src);
            }
#pragma unroll
            for (int q = 0; q < kStoreUnroll; ++q) {
                const int s = sb + q * R + o_s;
                const int64_t n = n0 + s;
                const float *row = o_tbl + static_cast<size_t>(ks[q]) * rs;
                float r[VEC];
                if constexpr (VEC % 4 == 0) {
#pragma unroll
                    for (int h = 0; h < VEC; h += 4) {
                        const float4 P = *reinterpret_cast<const float4 *>(row + h);
                        const float4 W = *reinterpret_cast<const float4 *>(row + Dw + h);
                        r[h] = fmaf(qs[q], W.x, P.x);
                        r[h + 1] = fmaf(qs[q], W.y, P.y);
                        r[h + 2] = fmaf(qs[q], W.z, P.z);
                        r[h + 3] = fmaf(qs[q], W.w, P.w);
                    }
                } else if constexpr (VEC == 2) {
                    // (8-byte LDS reads: Dw, the row stride and o_u * VEC are even)
                    const float2 P = *reinterpret_cast<const float2 *>(row);
                    const float2 W = *reinterpret_cast<const float2 *>(row + Dw);
                    r[0] = fmaf(qs[q], W.x, P.x);
                    r[1] = fmaf(qs[q], W.y, P.y);
                } else {
                    r[0] = fmaf(qs[q], row[Dw], row[0]);
                }
                const bool row_ok = o_ok && s < SW && n < n_end;
                emit_segment<Q, OUT, EPI, VEC, NT>(a, r, bvec, lwv, LIN ? xs[q] : 0.0f, row_ok,
                                               n * row_elems + static_cast<int64_t>(f0 + o_fl) * D + c0 + o_u * VEC,
                                               (n * F + f0 + o_fl) * a.MW, U, lane, o_u, m_shift, m_word);
            }
        }
    };

    // the early tiles from their registers (shifted down one a tile, so the
    // loop stays rolled), then the rest with the next tile's x loaded while
    // the current one is stored
    const int64_t t_rest = wave + static_cast<int64_t>(kXEarly) * kWaves;
    float v_next = load_x(t_rest);
    int64_t t = wave;
    for (int i = 0; i < kXEarly && t < n_tiles; ++i, t += kWaves) {
        const float v = x_early[0];
#pragma unroll
        for (int j = 0; j + 1 < kXEarly; ++j) x_early[j] = x_early[j + 1];
        tile(t, v);
    }
    for (; t < n_tiles; t += kWaves) {
        const float v = v_next;
        v_next = load_x(t + kWaves);
        tile(t, v);
    }
}

// ---------------------------------------------------------------------------
// wide tables
// ---------------------------------------------------------------------------

constexpr int kWideFB = 2 * kBlock;      // threads per wide-table workgroup
constexpr int kWideStage = 4096;         // weights staged per step of the prefix fold (16 KiB)

// One workgroup per (feature, sample chunk), for per-feature tables that do
// not fit LDS.  LDS holds the prefix at every S-th bin, cp[m][j] =
// sum_{i < m S} q(W[f, i, j]), folded in bin order from weights staged through
// LDS.  An output of bin k starts from cp[k / S] and adds q(W[f, i, j]) for
// i = S (k / S) .. k - 1 from global memory: the same fp32 additions in the
// same order as a fold from bin 0, hence the table kernel's bits.  Edges and
// inverse widths are in LDS when they fit (edges_lds), else the bin search
// reads them from global memory.  Stores, epilogues and ReLU bits as in the
// table kernel (one feature a group).
// find_bin over edges in global memory, with every es-th edge (es a power
// of two) in LDS: the sampled edges narrow the search to es - 1 edges, read
// from global memory.  For sorted edges the same bin as find_bin (the count
// of edges <= v, each level an upper bound); NaN walks to the top again.
__device__ __forceinline__ int find_bin_sampled(float v, const float *cs, int es_log, const float *e, int n) {
    const int nc = (n >> es_log) + 1;         // sampled edges 0, es, 2 es, ... <= n
    int lo = 0, hi = nc;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (v < cs[mid]) hi = mid;
        else lo = mid + 1;
    }
    // lo sampled edges are <= v: the count lies in [(lo - 1) es + 1, lo es]
    int k;
    if (lo == 0) {
        k = 0;
    } else {
        int a0 = ((lo - 1) << es_log) + 1;
        int b1 = min((lo << es_log) - 1, n) + 1;
        while (a0 < b1) {
            const int mid = (a0 + b1) >> 1;
            if (v < e[mid]) b1 = mid;
            else a0 = mid + 1;
        }
        k = a0 - 1;
    }
    k = k < 0 ? 0 : k;
    k = k > n - 1 ? n - 1 : k;
    return k;
}

template <int Q, int OUT, int EPI, int VEC, typename IdxT>
__global__ __launch_bounds__(kWideFB) void ple_fwd_wide_kernel(FwdArgs a) {
    constexpr int kWaves = kWideFB / kWave;
    constexpr bool HAS_BIAS = EPI == kEpiBias || EPI == kEpiBiasRelu;
    constexpr bool LIN = EPI == kEpiLin || EPI == kEpiLinRelu;
    extern __shared__ float smem[];
    const int B = a.B, D = a.D, F = a.F, S = a.S;
    float *cp = smem;                            // [ceil(B / S)][DC]
    float *stage = smem + a.stage_off;           // [kWideStage]
    float *sedge = smem + a.edge_off;            // [B + 1] (edges_lds), else [B / ES + 1] sampled edges
    float *siw = sedge + (B + 1);                // [B]     (edges_lds)

    int f, c;
    if (!decode_tile(blockIdx.x, a.G, a.C, f, c)) return;
    // column chunk of rows wider than a wave's lanes (as in the table kernel)
    const int cc = f % a.NCC;
    f /= a.NCC;
    const int c0 = cc * a.DC;
    const int Dw = min(a.DC, D - c0);
    const int64_t n_begin = static_cast<int64_t>(c) * a.NC;
    const int64_t n_end = min(a.N, n_begin + a.NC);
    if (n_begin >= n_end) return;
    const int tid = threadIdx.x;
    const int n = clamp_nbins(a.nbins[f], B);
    const float *wf = a.weight + static_cast<int64_t>(f) * B * D;
    const float *ef = a.edges + static_cast<int64_t>(f) * (B + 1);
    const float *iwf = a.iw + static_cast<int64_t>(f) * B;
    const int es_log = __ffs(a.ES) - 1;
    // dst[i] = get(i) for i < count, eight loads in flight per thread (a
    // plain loop waits for each load before the next)
    auto stage_lds = [&](float *dst, int count, auto get) __attribute__((always_inline)) {
        for (int i0 = tid; i0 < count; i0 += 8 * kWideFB) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = get(min(i0 + u * kWideFB, count - 1));
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (i0 + u * kWideFB < count) dst[i0 + u * kWideFB] = v[u];
        }
    };
    if (a.edges_lds) {
        // the search reads edges 0..n, the fraction inverse widths 0..n-1
        stage_lds(sedge, n + 1, [&](int i) { return ef[i]; });
        stage_lds(siw, n, [&](int i) { return iwf[i]; });
    } else {
        stage_lds(sedge, (n >> es_log) + 1, [&](int i) { return ef[i << es_log]; });
    }

    // ---- prefix checkpoints ------------------------------------------------
    // Weight rows 0..n-2 enter prefixes (the prefix of bin k sums bins < k,
    // all identity-mapped below the last bin).  Blocks of kb bins are staged
    // (contiguous rows of W); one lane per column turns the block in place
    // into its running prefix -- one chain of additions in bin order, the
    // LDS reads of eight steps ahead of them -- and then all threads copy
    // the block's checkpoints (bins that are multiples of S).
    const int kb = kWideStage / Dw;
    float acc = 0.0f;
    for (int k0 = 0; k0 < n; k0 += kb) {
        const int nk = min(kb, n - k0);
        const int nterm = min(nk, n - 1 - k0);       // rows of this block that enter a prefix
        stage_lds(stage, nk * Dw, [&](int i) {
            const int t = i / Dw;
            // (rows past the prefixes read row k0 and add zero)
            const float w = quant<Q>(wf[static_cast<int64_t>(k0 + (t < nterm ? t : 0)) * D + c0 + (i - t * Dw)]);
            return t < nterm ? w : 0.0f;
        });
        __syncthreads();
        if (tid < Dw) {
            int t0 = 0;
            for (; t0 + 16 <= nk; t0 += 16) {
                float v16[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) v16[u] = stage[(t0 + u) * Dw + tid];
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    stage[(t0 + u) * Dw + tid] = acc;
                    acc += v16[u];
                }
            }
            for (; t0 < nk; ++t0) {
                const float v = stage[t0 * Dw + tid];
                stage[t0 * Dw + tid] = acc;
                acc += v;
            }
        }
        __syncthreads();
        const int m_first = (k0 + S - 1) / S;
        const int m_end = (k0 + nk + S - 1) / S;   // checkpoints m S in [k0, k0 + nk)
        for (int i = tid; i < (m_end - m_first) * Dw; i += kWideFB) {
            const int mm = i / Dw;
            const int j = i - mm * Dw;
            cp[(m_first + mm) * Dw + j] = stage[((m_first + mm) * S - k0) * Dw + j];
        }
        __syncthreads();
    }

    // ---- stream wave tiles (one sample a lane, then rows of U lanes) -------
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int U = Dw / VEC;
    const int R = kWave / U;
    const float *e_row = a.edges_lds ? sedge : ef;
    const float *iw_row = a.edges_lds ? siw : iwf;
    const int o_s = lane / U;
    const int o_u = lane - o_s * U;
    const bool o_ok = o_s < R;
    float bvec[VEC], lwv[VEC];
#pragma unroll
    for (int t = 0; t < VEC; ++t) bvec[t] = lwv[t] = 0.0f;
    if constexpr (HAS_BIAS || LIN) {
        if (o_ok) {
            const int64_t pofs = static_cast<int64_t>(f) * D + c0 + o_u * VEC;
#pragma unroll
            for (int t = 0; t < VEC; ++t) {
                bvec[t] = HAS_BIAS ? a.bias[pofs + t] : a.lin_b[pofs + t];
                if constexpr (LIN) lwv[t] = a.lin_w[pofs + t];
            }
        }
    }
    const int m_shift = (o_u * VEC) & 31;
    const int m_word = (o_u * VEC) >> 5;
    const float *wcol = wf + c0 + o_u * VEC;       // this lane's columns of W[f]
    const int64_t rows = n_end - n_begin;
    const int64_t n_tiles = (rows + kWave - 1) / kWave;
    const int64_t row_elems = static_cast<int64_t>(F) * D;

    for (int64_t t = wave; t < n_tiles; t += kWaves) {
        const int64_t n0 = n_begin + t * kWave;
        const int64_t pn = n0 + lane;
        const bool pvalid = pn < n_end;
        const float v = pvalid ? a.x[pn * F + f] : 0.0f;
        const int k = a.edges_lds ? find_bin(v, e_row, n) : find_bin_sampled(v, sedge, es_log, ef, n);
        const float qf = quant<Q>((v - e_row[k]) * iw_row[k]);
        if (pvalid && cc == 0) static_cast<IdxT *>(a.idx)[pn * F + f] = static_cast<IdxT>(k);

        for (int sb = 0; sb < kWave; sb += R) {
            const int s = sb + o_s;
            const int src = s & (kWave - 1);
            const int ks = __shfl(k, src);
            const float qs = __shfl(qf, src);
            const float xs = LIN ? __shfl(v, src) : 0.0f;
            const int64_t nn = n0 + s;
            const bool row_ok = o_ok && s < kWave && nn < n_end;
            float r[VEC];
            if (row_ok) {
                const int m = ks / S;
                float P[VEC], W[VEC];
                lds_load_vec<VEC>(cp + m * Dw + o_u * VEC, P);
                // the rows between the checkpoint and the bin, eight loads
                // ahead of their additions (in bin order)
                for (int i0 = m * S; i0 < ks; i0 += 8) {
                    float w8[8][VEC];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const float *wi = wcol + static_cast<int64_t>(min(i0 + u, ks - 1)) * D;
#pragma unroll
                        for (int h = 0; h < VEC; ++h) w8[u][h] = wi[h];
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        if (i0 + u < ks) {
#pragma unroll
                            for (int h = 0; h < VEC; ++h) P[h] += quant<Q>(w8[u][h]);
                        }
                    }
                }
                const float *wk = wcol + static_cast<int64_t>(phys_bin(ks, n, B)) * D;
#pragma unroll
                for (int h = 0; h < VEC; ++h) W[h] = quant<Q>(wk[h]);
#pragma unroll
                for (int h = 0; h < VEC; ++h) r[h] = fmaf(qs, W[h], P[h]);
            } else {
#pragma unroll
                for (int h = 0; h < VEC; ++h) r[h] = 0.0f;
            }
            emit_segment<Q, OUT, EPI, VEC>(a, r, bvec, lwv, xs, row_ok, nn * row_elems + static_cast<int64_t>(f) * D + c0 + o_u * VEC,
                                           (nn * F + f) * a.MW, U, lane, o_u, m_shift, m_word);
        }
    }
}

// LDS per workgroup the planner aims for: small tables keep many workgroups
// (and their loads) in flight per CU, which the store stream needs more than
// wide feature groups.  (Measured at F=128, 48 bins, d=32: two features per
// workgroup, 25 KB, beat one by 3-11 us; four, 50 KB, lost 15-40 us.)
constexpr size_t kLdsBudget = 32 * 1024;
// Each workgroup writes at least this many times the table bytes it stages
// (see plan_forward).
constexpr int kOutPerTable = 10;

struct FwdPlan {
    int vec, FS, G, C, FB;
    int DC = 0, NCC = 1;                // column chunks (rows wider than a wave's lanes)
    int64_t NC;
    size_t lds;
    bool wide = false;                  // ple_fwd_wide_kernel
    int S = 1, stage_off = 0, edge_off = 0, edges_lds = 0, ES = 1;
};

// Wide tables: the prefix checkpoints take at most kWideCpBudget bytes of
// LDS (the smallest stride S that fits), the edges and inverse widths join
// them when they fit kWideEdgeBudget.
constexpr size_t kWideCpBudget = 96 * 1024;
constexpr size_t kWideEdgeBudget = 40 * 1024;
constexpr size_t kWideSampleBudget = 16 * 1024;

// Rows of more than a wave's lanes (D / vec > 64) are cut into NCC chunks of
// DC columns (a multiple of vec), as even as the lanes allow.
void plan_chunks(int64_t D, FwdPlan &pl) {
    const int64_t U = D / pl.vec;
    pl.NCC = static_cast<int>((U + kWave - 1) / kWave);
    pl.DC = static_cast<int>((U + pl.NCC - 1) / pl.NCC) * pl.vec;
}

void plan_wide(int64_t N, int64_t F, int64_t B, int64_t D, int out_bytes, FwdPlan &pl) {
    pl.wide = true;
    pl.FS = 1;
    pl.FB = kWideFB;
    if (pl.vec == 8) pl.vec = 4;
    plan_chunks(D, pl);
    const int64_t Dc = pl.DC;
    int64_t S = (B * Dc * 4 + static_cast<int64_t>(kWideCpBudget) - 1) / static_cast<int64_t>(kWideCpBudget);
    if (S < 1) S = 1;
    const int64_t ncp = (B + S - 1) / S;
    pl.S = static_cast<int>(S);
    pl.stage_off = static_cast<int>(align_up(static_cast<size_t>(ncp * Dc), 4));
    pl.edge_off = pl.stage_off + kWideStage;
    pl.edges_lds = static_cast<size_t>(2 * B + 1) * 4 <= kWideEdgeBudget ? 1 : 0;
    // otherwise every ES-th edge, ES the smallest power of two (at least 8)
    // whose samples fit kWideSampleBudget
    pl.ES = 1;
    if (!pl.edges_lds) {
        pl.ES = 8;
        while (static_cast<size_t>(B / pl.ES + 1) * 4 > kWideSampleBudget) pl.ES *= 2;
    }
    const size_t edge_floats = pl.edges_lds ? static_cast<size_t>(2 * B + 1) : static_cast<size_t>(B / pl.ES + 1);
    pl.lds = 4 * (static_cast<size_t>(pl.edge_off) + edge_floats);
    pl.G = static_cast<int>(F) * pl.NCC;
    // chunks: one round of the workgroups the CUs hold at once (LDS), so
    // every workgroup folds its prefix at the same time; the weights a fold
    // reads again per chunk come from the caches
    // (PLE_TUNE_FWD_WG_PER_CU: that many per CU)
    const int wg_env = tuning(PLE_TUNE_FWD_WG_PER_CU);
    const int64_t resident = std::max<int64_t>(1, static_cast<int64_t>(kLdsMax / pl.lds));
    const int64_t target = (wg_env > 0 ? wg_env : resident) * device_cu_count();
    int64_t c = (target + pl.G - 1) / pl.G;
    const int64_t max_c = (N + kWave - 1) / kWave;
    if (c > max_c) c = max_c;
    if (c < 1) c = 1;
    pl.NC = (N + c - 1) / c;
    pl.C = static_cast<int>((N + pl.NC - 1) / pl.NC);
}

// FS: the widest power-of-two feature group whose row fits one wave's stores
// (FS * D/VEC <= 64) and whose tables fit kLdsBudget; then, while a sample's
// segment of the group (FS * D outputs) is shorter than a 128-byte line, wider
// up to the LDS limit -- partial lines written by different workgroups at
// different times cost more than the LDS.
// Chunks: about 32 workgroups per CU over the grid, but each workgroup writes
// at least kOutPerTable times its tables' bytes, since the table staging and
// the prefix pass are paid per workgroup.  Together, measured: c2 131 -> 59
// us, c3 186 -> 155 us, c4 517 -> 221 us, c1 unchanged (its plan is the same).
// PLE_TUNE_FWD_FS / PLE_TUNE_FWD_WG_PER_CU override the two choices.

// out16: the output's base address is 16-byte aligned (8 outputs per lane);
// relu: the epilogue writes ReLU pass bits
bool plan_forward(int64_t N, int64_t F, int64_t B, int64_t D, int out_bytes, bool aligned16, bool out16, bool relu,
                  FwdPlan &pl) {
    // 16-bit outputs: 8 per lane (one 16-byte store) when D allows, so a
    // store instruction carries as many bytes as fp32's 4 per lane
    // Even D not a multiple of 4: 2 per lane (8-byte stores), half the store
    // instructions and table reads of one per lane
    pl.vec = (D % 4 == 0 && aligned16) ? 4 : ((D % 2 == 0 && aligned16 && tuning(PLE_TUNE_FWD_VEC) != 1) ? 2 : 1);
    if (out_bytes == 2 && D % 8 == 0 && aligned16 && out16 && tuning(PLE_TUNE_FWD_VEC) != 4) pl.vec = 8;
    plan_chunks(D, pl);
    // Tables beyond LDS: rows cut into narrower column chunks (one feature a
    // group) until a chunk's tables fit, while a chunk's segment of a row
    // keeps 64 bytes, before the wide-table kernel.  At N = 65536, fp32:
    // B = 1024, d = 32 (two chunks of 16) 601 -> 328 us, B = 700, d = 64
    // (three of 24 or 16) 567 -> 504 us; B = 2048, d = 16 (two of 8, 32-byte
    // segments) 137 -> 159 us, so not there.  (Not with a ReLU: a row's pass
    // bits are gathered from the lanes of one chunk.)
    if (!relu && tuning(PLE_TUNE_FWD_WIDE) != 1) {
        const int64_t U = D / pl.vec;
        int64_t ncc = pl.NCC;
        FwdPlan t = pl;
        while (fwd_lds_bytes(1, B, t.DC) > kLdsMax && t.DC > t.vec) {
            ++ncc;
            const int64_t dcu = (U + ncc - 1) / ncc;
            t.DC = static_cast<int>(dcu * t.vec);
            t.NCC = static_cast<int>((U + dcu - 1) / dcu);
        }
        if (t.DC * out_bytes >= 64 || t.NCC == pl.NCC) pl = t;
    }
    if (fwd_lds_bytes(1, B, pl.DC) > kLdsMax || tuning(PLE_TUNE_FWD_WIDE) == 1) {
        plan_wide(N, F, B, D, out_bytes, pl);
        return true;
    }
    // (rows of several chunks: one feature a group; D below is a chunk's width)
    const int U = pl.DC / pl.vec;
    const int Bi = static_cast<int>(B), Di = pl.DC;
    auto fits_wave = [&](int f) {
        return f <= kWave && f * U <= kWave && (f == 1 || f / 2 < F) && (f == 1 || pl.NCC == 1);
    };
    int fs = 1;
    while (fits_wave(fs * 2) && fwd_lds_bytes(fs * 2, Bi, Di) <= kLdsBudget) fs *= 2;
    // Rows of up to 24 columns run 512-thread workgroups (below), whose waves
    // share one table: twice the budget, up to 8 features, while at least 16
    // feature groups remain (d = 24: 175 -> 155 us, d = 12: 86 -> 82 us,
    // d = 14: 172 -> 163 us at F=128, 48 bins, N=65536; d = 16 within noise;
    // 16 features at d = 8 lost 17 us, 4 at F = 8 (c0) 2 us)
    if (D <= 24)
        while (fs < 8 && fits_wave(fs * 2) && fwd_lds_bytes(fs * 2, Bi, Di) <= 2 * kLdsBudget &&
               F >= 16 * 2 * fs)
            fs *= 2;
    // A single feature a group (wide D): two features within twice the
    // budget (at F=128, 48 bins, N=65536: d = 44 856 -> 502 us, d = 48 372 ->
    // 298 us, d = 50 650 -> 450 us, d = 56 793 -> 372 us, d = 62 741 -> 544
    // us, d = 64 390 -> 340 us)
    if (fs == 1 && fits_wave(2) && fwd_lds_bytes(2, Bi, Di) <= 2 * kLdsBudget) fs = 2;
    while (static_cast<int64_t>(fs) * Di * out_bytes < 128 && fits_wave(fs * 2) &&
           fwd_lds_bytes(fs * 2, Bi, Di) <= kLdsMax)
        fs *= 2;
    const int fs_env = tuning(PLE_TUNE_FWD_FS);
    if (fs_env > 0 && (fs_env & (fs_env - 1)) == 0 && fits_wave(fs_env) &&
        fwd_lds_bytes(fs_env, Bi, Di) <= kLdsMax)
        fs = fs_env;
    pl.lds = fwd_lds_bytes(fs, Bi, Di);
    if (pl.lds > kLdsMax) return false;
    // 512 threads where the tables leave room for two workgroups per CU or
    // fewer, and for rows of up to 24 columns: the extra waves hide the bin
    // search's dependent LDS reads, which weigh more the fewer bytes a pair
    // writes, and each table is staged for twice as many of them.  Measured
    // (F=128, 48 bins, N=65536 unless named): c4 204 -> 151 us, c3 157 -> 125
    // us, d=12 97 -> 86 us, d=24 184 -> 175 us; d=32 (c1) and d=48 the same,
    // d=64 +7 us.  PLE_TUNE_FWD_FB overrides it.
    pl.FB = (kLdsMax / pl.lds < 3 || Di <= 24) ? 2 * kBlock : kBlock;
    const int fb_env = tuning(PLE_TUNE_FWD_FB);
    if (fb_env == kBlock || fb_env == 2 * kBlock) pl.FB = fb_env;
    pl.FS = fs;
    pl.G = static_cast<int>((F + fs - 1) / fs) * pl.NCC;
    const int wg_env = tuning(PLE_TUNE_FWD_WG_PER_CU);
    const int64_t target = static_cast<int64_t>(wg_env > 0 ? wg_env : 32) * device_cu_count();
    int64_t c = (target + pl.G - 1) / pl.G;
    if (wg_env <= 0) {
        // output per workgroup (NC * FS * D * out_bytes) >= kOutPerTable * tables (FS * B * D * 4)
        const int64_t min_nc = (static_cast<int64_t>(kOutPerTable) * B * 4 + out_bytes - 1) / out_bytes;
        const int64_t c_tbl = (N + min_nc - 1) / min_nc;
        if (c > c_tbl) c = c_tbl;
        // Tables that leave room for at most two workgroups per CU: exactly
        // two rounds of resident workgroups, so the last round is as full as
        // the first (fwd+bwd step, its forward: c3 156 -> 140 us, c2 58 -> 57
        // us, c4 165 -> 159 us, against 1.6 to 3.2 rounds before)
        if (kLdsMax / pl.lds <= 2) {
            const int64_t slots = static_cast<int64_t>(kLdsMax / pl.lds) * device_cu_count();
            c = (2 * slots) / pl.G;
            // 16-bit outputs: one round -- a workgroup writes half the bytes
            // per pair, so its table staging and prefix pass weigh twice as
            // much (c4's forward in the fwd+bwd step: 131 -> 120 us; c2 / c3,
            // fp32, keep two rounds: one costs them 3 us)
            if (out_bytes == 2) c = slots / pl.G;
            if (c < 1) c = 1;
        }
    }
    const int64_t sw = kWave / fs;
    const int64_t max_c = (N + sw - 1) / sw;          // at least one wave tile per chunk
    if (c > max_c) c = max_c;
    if (c < 1) c = 1;
    pl.NC = (N + c - 1) / c;
    pl.C = static_cast<int>((N + pl.NC - 1) / pl.NC);
    return true;
}

// Timer events of the forward launch being issued (forward_run sets them;
// both NULL unless kernel timing is on).
thread_local TimerSlot t_slot;

template <typename K>
void launch_fwd(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, const FwdArgs &a) {
    hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), s, t_slot.start, t_slot.stop, 0u, a);
}

// the table kernel, with plain output stores where the launch asks for them
// and the instantiation would stream (out_nt)
template <int Q, int OUT, int EPI, int VEC, typename IdxT, int FB>
void launch_tbl(const FwdArgs &a, dim3 grid, size_t lds, hipStream_t s) {
    constexpr bool kHasNT = OUT == PLE_DTYPE_F32 ? VEC >= 4 : VEC >= 2;
    if constexpr (kHasNT) {
        if (!a.out_nt) {
            launch_fwd((ple_fwd_kernel<Q, OUT, EPI, VEC, IdxT, FB, false>), grid, dim3(FB), lds, s, a);
            return;
        }
    }
    launch_fwd((ple_fwd_kernel<Q, OUT, EPI, VEC, IdxT, FB>), grid, dim3(FB), lds, s, a);
}

template <int Q, int OUT, int EPI, int VEC>
hipError_t launch_idx(const FwdArgs &a, int idxb, bool wide, dim3 grid, size_t lds, hipStream_t s) {
    // uint8 indices up to 256 bins, int16 up to 32768, int32 beyond (those
    // tables never fit the table kernel's LDS)
    if (wide) {
        if (idxb == 1) launch_fwd((ple_fwd_wide_kernel<Q, OUT, EPI, VEC, uint8_t>), grid, dim3(kWideFB), lds, s, a);
        else if (idxb == 2) launch_fwd((ple_fwd_wide_kernel<Q, OUT, EPI, VEC, int16_t>), grid, dim3(kWideFB), lds, s, a);
        else launch_fwd((ple_fwd_wide_kernel<Q, OUT, EPI, VEC, int32_t>), grid, dim3(kWideFB), lds, s, a);
        return hipGetLastError();
    }
    if (idxb == 4) return hipErrorInvalidConfiguration;
    if (a.FB == 2 * kBlock) {
        if (idxb == 1) launch_tbl<Q, OUT, EPI, VEC, uint8_t, 2 * kBlock>(a, grid, lds, s);
        else launch_tbl<Q, OUT, EPI, VEC, int16_t, 2 * kBlock>(a, grid, lds, s);
    } else {
        if (idxb == 1) launch_tbl<Q, OUT, EPI, VEC, uint8_t, kBlock>(a, grid, lds, s);
        else launch_tbl<Q, OUT, EPI, VEC, int16_t, kBlock>(a, grid, lds, s);
    }
    return hipGetLastError();
}

template <int Q, int OUT, int EPI>
hipError_t launch_vec(const FwdArgs &a, int vec, int idxb, bool wide, dim3 grid, size_t lds, hipStream_t s) {
    // (8 outputs per lane: 16-bit outputs without an epilogue, table kernel only)
    if constexpr (OUT != PLE_DTYPE_F32 && EPI == kEpiNone) {
        if (vec == 8 && !wide) {
            if (a.FB == 2 * kBlock) {
                if (idxb == 1) launch_tbl<Q, OUT, EPI, 8, uint8_t, 2 * kBlock>(a, grid, lds, s);
                else launch_tbl<Q, OUT, EPI, 8, int16_t, 2 * kBlock>(a, grid, lds, s);
            } else {
                if (idxb == 1) launch_tbl<Q, OUT, EPI, 8, uint8_t, kBlock>(a, grid, lds, s);
                else launch_tbl<Q, OUT, EPI, 8, int16_t, kBlock>(a, grid, lds, s);
            }
            return hipGetLastError();
        }
    }
    if (vec == 4) return launch_idx<Q, OUT, EPI, 4>(a, idxb, wide, grid, lds, s);
    if (vec == 2) return launch_idx<Q, OUT, EPI, 2>(a, idxb, wide, grid, lds, s);
    return launch_idx<Q, OUT, EPI, 1>(a, idxb, wide, grid, lds, s);
}

// Supported (quant, output) pairs: output == quant without an epilogue (the
// reference operator), output == F32 with one (the fused module tail).
template <int Q>
hipError_t launch_q(const FwdArgs &a, int epi, int vec, int idxb, bool wide, dim3 grid, size_t lds, hipStream_t s) {
    switch (epi) {
        case kEpiBias: return launch_vec<Q, PLE_DTYPE_F32, kEpiBias>(a, vec, idxb, wide, grid, lds, s);
        case kEpiBiasRelu: return launch_vec<Q, PLE_DTYPE_F32, kEpiBiasRelu>(a, vec, idxb, wide, grid, lds, s);
        case kEpiLin: return launch_vec<Q, PLE_DTYPE_F32, kEpiLin>(a, vec, idxb, wide, grid, lds, s);
        case kEpiLinRelu: return launch_vec<Q, PLE_DTYPE_F32, kEpiLinRelu>(a, vec, idxb, wide, grid, lds, s);
        default: return launch_vec<Q, Q, kEpiNone>(a, vec, idxb, wide, grid, lds, s);
    }
}

}  // namespace

int forward_run(const ForwardRequest &r) {
    // epilogue: bias (+ ReLU) or linear0 (+ ReLU); never both, ReLU needs one
    if (r.bias && r.lin_w) return PLE_E_UNSUPPORTED;
    if (r.lin_w && !r.lin_b) return PLE_E_NULL_POINTER;
    if (r.relu && !r.bias && !r.lin_w) return PLE_E_UNSUPPORTED;
    // module epilogues with ReLU or linear0: rows of at most 64 columns (the
    // module's limit on d_embedding; the ReLU pass bits are gathered from one
    // row's lanes)
    if ((r.relu || r.lin_w) && r.D > 64) return PLE_E_TOO_LARGE;
    const int epi = r.bias ? (r.relu ? kEpiBiasRelu : kEpiBias)
                  : r.lin_w ? (r.relu ? kEpiLinRelu : kEpiLin) : kEpiNone;
    if (epi != kEpiNone ? r.out_dtype != PLE_DTYPE_F32 : r.out_dtype != r.quant) return PLE_E_UNSUPPORTED;
    const int out_bytes = r.out_dtype == PLE_DTYPE_F32 ? 4 : 2;
    if (reinterpret_cast<uintptr_t>(r.out) % out_bytes != 0) return PLE_E_MISALIGNED;
    const bool aligned16 = (reinterpret_cast<uintptr_t>(r.out) % (4 * out_bytes) == 0) &&
                           (reinterpret_cast<uintptr_t>(r.weight) % 16 == 0);
    FwdPlan pl;
    if (!plan_forward(r.N, r.F, r.B, r.D, out_bytes, aligned16, reinterpret_cast<uintptr_t>(r.out) % 16 == 0,
                      r.relu != 0, pl))
        return PLE_E_UNSUPPORTED;
    FwdArgs a;
    a.x = r.x; a.edges = r.edges; a.iw = r.iw; a.nbins = r.nbins; a.weight = r.weight;
    a.bias = r.bias; a.lin_w = r.lin_w; a.lin_b = r.lin_b;
    a.mask = r.relu ? r.mask : nullptr; a.MW = static_cast<int>((r.D + 31) / 32);
    a.out = r.out; a.idx = r.idx;
    a.N = r.N; a.F = static_cast<int>(r.F); a.B = static_cast<int>(r.B); a.D = static_cast<int>(r.D);
    a.FS = pl.FS; a.G = pl.G; a.C = pl.C; a.NC = pl.NC; a.FB = pl.FB;
    a.DC = pl.DC; a.NCC = pl.NCC;
    // A feature group's outputs of a sample are one segment of FS * D
    // outputs; the neighbouring group writes the rest of its first and last
    // lines.  Streaming stores suit segments whose ends fall on 64-byte
    // boundaries; at other ends the partial writes reach memory unmerged,
    // and plain stores let the L2 of the XCD, which runs both groups, merge
    // the lines first (F = 128, 48 bins, N = 65536: d = 28 fp32 380 -> 298 us,
    // d = 44 504 -> 409 us; at 64-byte ends plain stores lost 15-35%).
    {
        const int64_t seg = static_cast<int64_t>(pl.FS) * pl.DC * out_bytes;
        const int64_t row = r.F * r.D * out_bytes;
        a.out_nt = seg % 64 == 0 && row % 64 == 0 && reinterpret_cast<uintptr_t>(r.out) % 64 == 0;
    }
    a.S = pl.S; a.stage_off = pl.stage_off; a.edge_off = pl.edge_off; a.edges_lds = pl.edges_lds; a.ES = pl.ES;
    const int64_t grid = kNumXcd * tiles_per_xcd(pl.G, pl.C);
    if (grid > INT32_MAX) return PLE_E_TOO_LARGE;
    const int idxb = idx_bytes_for(r.B);
    hipError_t e;
    t_slot = timer_slot(PLE_TIMER_FORWARD);
    switch (r.quant) {
        case PLE_DTYPE_F32: e = launch_q<PLE_DTYPE_F32>(a, epi, pl.vec, idxb, pl.wide, dim3(grid), pl.lds, r.stream); break;
        case PLE_DTYPE_F16: e = launch_q<PLE_DTYPE_F16>(a, epi, pl.vec, idxb, pl.wide, dim3(grid), pl.lds, r.stream); break;
        default: e = launch_q<PLE_DTYPE_BF16>(a, epi, pl.vec, idxb, pl.wide, dim3(grid), pl.lds, r.stream); break;
    }
    if (e == hipSuccess) timer_commit(t_slot);
    t_slot = TimerSlot{};
    return e == hipSuccess ? PLE_OK : static_cast<int>(e);
}

}  // namespace ple
