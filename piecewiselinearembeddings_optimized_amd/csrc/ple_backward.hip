// Backward kernels of the fused PLE path (gfx950).
//
// dx[n,f]  = iw_k <g, q(W[f,phys(k)])> (+ iw_{k-1} <g, q(W[f,k-1])> when
//            k > 0 and x == e_k)                  reference backward_cuda.cu:380-490
// dW[f,phys(k)] = sum_{bin=k} q(frac) g + sum_{bin>k} g
//                                                 reference backward_cuda.cu:170-336,889-923
// db[f]    = sum_n g                              (autograd of module.py:238-239)
//
// Module epilogues (the backward of the fused forward tails, module.py:230-248;
// the gradient is then fp32):
//   ReLU      g_ple = g * pass[n, f, j] (the forward's bits); with a bias,
//             db = sum_n g_ple
//   linear0   g_ple = g (or g * pass with ReLU); dx += <g, lin_w[f]>,
//             d lin_w[f] = sum_n g x, d lin_b[f] = sum_n g (in db's slot)
// dx and dW use g_ple rounded through the quantisation dtype.
//
// Main path: ple_bwd_fused_kernel, over tiles of P (sample, feature) pairs
// (NT samples x FS features, "sub-tiles").  One workgroup per feature group
// and chunk of SPC sub-tiles; every thread takes part in both jobs, which
// interleave sub-tile by sub-tile:
//
// sort -- the bin index and x of every pair of the next sub-tile (loaded a
//   sub-tile ahead) give q(frac) and the edge flag; a counting sort by
//   (feature, bin): per 64-pair block, ranks of equal keys from 64-bit
//   ballots plus the key's count in the block, then a scan over the keys --
//   deterministic and stable.  It writes the sorted row descriptors
//   {q(frac) (-0 marks x on the bin's left edge), sample | feature << 24} and
//   the sub-tile's pieces: every (feature, bin) run of sorted rows cut into
//   pieces of kL rows.  Nothing leaves LDS.
//
// reduce -- the gradient stream and LDS work.  Lane groups (D/VEC lanes, one
//   grad_output row per step) take equal runs of pieces: each row is read
//   once, its dx is the lane group's DPP-reduced dot with the LDS weight row
//   (kept in the row's descriptor once the row is reduced), and bucket /
//   weighted / bias sums run in registers until the key changes (checked
//   once per piece).  A run's first key goes to a per-run record, every later
//   key straight into the LDS histogram (no other run can own it); the
//   records are added run by run in order.  The sub-tile's dx leaves from
//   the descriptors straight into dx [N, F].  The chunk's histogram is
//   written once.
//
// ple_bwd_chunksum_kernel adds the chunk partials in chunk order;
// ple_bwd_finalize_kernel takes the suffix over bins.
//
// No floating-point atomics anywhere, a fixed order for every sum, so results
// repeat bitwise.
//
// Fallback (shapes whose tables do not fit the sorted path's LDS, any number
// of bins): ple_bwd_simple_dx_kernel and ple_bwd_simple_hist_kernel (cells in
// LDS, or in the partials in global memory when B * D * 8 bytes exceed LDS),
// same partial layout, same finalize.

#include <algorithm>

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
    float *part;     // [Cd][F][B][2D] chunk partials {bucket | weighted}
    float *part_db;  // [Cd][F][D] chunk partials of the bias gradient
    const uint32_t *mask;   // [N][F][MW] ReLU pass bits of the forward (epilogue with ReLU)
    const float *lin_w;     // [F][D] linear0 weight (version-B epilogue)
    float *part_lw;         // [Cd][F][D] chunk partials of the linear0 weight gradient
    float *dlw;             // [F][D] linear0 weight gradient
    int MW;                 // mask words per (sample, feature) row
    int64_t N;
    int F, B, D;
    int C;           // chunks (fallback: of samples; sorted path: of sub-tiles)
    int Cd;          // chunks holding samples (the ones that write partials)
    int64_t NC;      // fallback: samples per chunk
    int db_from_buckets;   // finalize: db = sum of the bin buckets (no raw-gradient partials)
    int fin_direct;        // finalize: chunk sums read straight from the partials (no LDS table)
    int fin_summed;        // finalize: the chunk partials are summed into chunk 0 already
    int fin_fused;         // sorted path, one chunk: dW / db straight from the LDS histogram (no finalize kernel)
    int idxb;              // bytes per bin index
    // sorted path
    int FS, G, NT, T, SPC, PM, LGW;   // T sub-tiles, SPC sub-tiles per chunk, PM piece capacity
    // Bin windows: a workgroup holds the tables and histogram cells of BW
    // consecutive bins of its features (BW = B, NW = 1 when every bin fits
    // in LDS); the NW windows of a feature group are NW workgroups, and
    // each pair is reduced (and its dx written) by the window of its bin.
    int BW, NW;
    int ro_qw, ro_hist, ro_db, ro_iw, ro_nb, ro_desc, ro_piece, ro_npc, ro_rec, ro_rkey, ro_rfl, ro_dx,
        ro_lw, ro_dlw, ro_xs, ro_edge, ro_cnt, ro_seg, ro_tmp;   // fused kernel LDS (ro_dx < 0: no dx staging;
                                                                  // matrix-core kernel: ro_tmp its non-finite records)
};

constexpr int kP = 1024;                        // (sample, feature) pairs per sub-tile
// Rows per piece: every (feature, bin) run of a sorted sub-tile is cut into
// pieces of kL consecutive rows (the last one shorter).
constexpr int kL = 4;

// backward epilogue flags (template argument of the reduce kernel)
// Reduce workgroups of twice the usual size: where LDS leaves room for only
// one reduce workgroup per CU, its waves are all the CU has to hide latency.
constexpr int kWideBlock = 2 * kBlock;

constexpr int kBwdRelu = 1;
constexpr int kBwdLin = 2;
// (not an epilogue) gradient rows that end inside a 128-byte line: plain
// loads where the lane group's width would stream them.  Rows of d = 24
// fp32 (96 bytes): backward 367 -> 304 us at N = 65536, F = 128, 48 bins;
// d = 32 (whole lines) keeps the streaming loads (286 us; 306 us plain).
constexpr int kBwdShared = 4;

// finalize (dW / db from the chunk partials): one workgroup per (feature,
// group of kFinCols columns), kFinLanes lanes per column
constexpr int kFinCols = 8;
// LDS row stride of the chunk-sum table: one more than kFinCols, so that the
// lanes of a column (consecutive bins) read distinct banks
constexpr int kFinStride = kFinCols + 1;
constexpr int kFinLoadsInline = 128;   // chunk-sum loads per finalize thread, at most
constexpr int kFinLanes = kBlock / kFinCols;   // lanes per column (half a wave)
constexpr int kFinBatch = 8;                     // partial-sum elements a finalize thread loads together

// One column's dW from its per-bin sums, by kFinLanes lanes (l: this lane's
// place among them): each lane sums the buckets of its run of the n bins, a
// suffix scan over the lanes gives every run the sum of the runs above it,
// and each lane walks its run from the top, dW[phys k] = weighted[k] +
// sum_{m > k} bucket[m]; slots no bin maps to get 0.  total(k, h): bin k's
// bucket (h = 0) or weighted (h = 1) sum; dw: the column's dW (stride D
// between slots) or null.  Returns the lanes' running sums: lane 0 holds the
// column's bucket total.  Every lane of the group takes part (a lane with
// n = 0 adds zeros), so the shuffles see live lanes.  A fixed order: results
// repeat bitwise.  LANES: lanes a column (a power of two up to a wave).
template <int LANES = kFinLanes, typename Total>
__device__ __forceinline__ float dw_suffix(Total total, int n, int B, int D, int l, float *dw) {
    const int m = (n + LANES - 1) / LANES;   // bins per lane
    const int lo = min(n, l * m);
    const int hi = min(n, lo + m);
    float run = 0.0f;
#pragma unroll 4
    for (int k = hi - 1; k >= lo; --k) run += total(k, 0);
    // inclusive suffix over the lanes: sum of the runs of lanes l, l+1, ...
    float incl = run;
#pragma unroll
    for (int off = 1; off < LANES; off <<= 1) {
        const float t = __shfl_down(incl, off, LANES);
        if (l + off < LANES) incl += t;
    }
    const float above = __shfl_down(incl, 1, LANES);
    if (dw) {
        float fut = l + 1 < LANES ? above : 0.0f;
#pragma unroll 4
        for (int k = hi - 1; k >= lo; --k) {
            dw[static_cast<int64_t>(phys_bin(k, n, B)) * D] = total(k, 1) + fut;
            fut += total(k, 0);
        }
        for (int k = n - 1 + l; k < B - 1; k += LANES) dw[static_cast<int64_t>(k) * D] = 0.0f;
    }
    return incl;
}

// ---------------------------------------------------------------------------
// sub-tile sort (all threads of the fused kernel, between reduce phases)
// ---------------------------------------------------------------------------

constexpr int kBlocks = kP / kWave;   // 64-pair blocks of a sub-tile

// uint16 block counts per block row: NK keys, padded to whole dwords
__host__ __device__ __forceinline__ int cnt_stride(int NK) { return (NK + 1) & ~1; }

// Bin index and x of this thread's pairs of sub-tile t: pairs p = tid + u RB
// in sample-major order (p = s * FS + fl), so a load instruction covers whole
// runs of each sample's features.  Pairs outside the batch or the feature
// range read pair 0 (ignored when sorted).
template <int RB, typename IdxT>
__device__ __forceinline__ void tile_load(const BwdArgs &a, int t, int f0, int nfh, int tid, int (&pk)[kP / RB],
                                          float (&pv)[kP / RB]) {
    const int FS = a.FS;
    const int fs_shift = __ffs(FS) - 1;
    const int64_t sub = static_cast<int64_t>(t) * a.NT;
    const int ns = static_cast<int>(min(static_cast<int64_t>(a.NT), a.N - sub));
#pragma unroll
    for (int u = 0; u < kP / RB; ++u) {
        const int p = tid + u * RB;
        const int s = p >> fs_shift;
        const int fl = p & (FS - 1);
        const int64_t pair = (s < ns && fl < nfh) ? (sub + s) * a.F + f0 + fl : 0;
        pk[u] = load_idx<IdxT>(a.idx, pair);
        pv[u] = a.x[pair];
    }
}

// Counting sort of sub-tile t's pairs by key (feature, bin) = fl * B + bin,
// stable and deterministic, by all RB threads, in two parts:
// tile_rank (A), then -- after a barrier -- tile_place (B, C):
//   A. per pair: bin, q(frac) and the edge flag; its rank among the equal
//      keys of its 64-pair block (64-bit ballots over the bin bits within the
//      lanes of its feature -- a lane's feature is the same in every block);
//      the block's first pair of each key stores the key's count in the block
//      (s_cnt, whose row the ranking wave zeroes first).  Per pair
//      key | rank << 16 and the q(frac) bits stay in registers.
//   B. per key (each thread a contiguous run of keys): the exclusive prefix
//      of its block counts in place, then a scan over the keys gives every key
//      its first row and first piece (pieces: the key's rows cut into runs of
//      kL) in s_seg, with the totals in s_seg[NK];
//   C. scatter: row descriptor {q(frac) bits (-0: x on the bin's left edge,
//      k >= 1; a real -0 is stored as +0), sample | fl << 24} at its sorted
//      position, and the piece entry {bin | fl << 12 | first row << 16 |
//      (rows - 1) << 28} from each piece's first row.
// Pairs outside the batch or feature range take key NK and are not stored.
// The caller synchronises between the parts, before the descriptors are
// read, and between this sort's part B / C and the next sort's part A (one
// count buffer).
template <int Q, int RB>
__device__ __forceinline__ void tile_rank(const BwdArgs &a, int t, int k0, int nfh, int tid, const int (&pk)[kP / RB],
                                          const float (&pv)[kP / RB], const int *s_nb, const float *s_edge,
                                          const float *s_iw, uint16_t *s_cnt, int (&ko)[kP / RB],
                                          uint32_t (&qb)[kP / RB]) {
    constexpr int kPR = kP / RB;
    const int FS = a.FS, B = a.BW, NT = a.NT;    // (B: the window's bins)
    const int fs_shift = __ffs(FS) - 1;
    const int ns = static_cast<int>(min(static_cast<int64_t>(NT), a.N - static_cast<int64_t>(t) * NT));
    const int NK = FS * B;                       // keys; NK marks padding
    const int lane = tid & (kWave - 1);
    const int fl = lane & (FS - 1);              // this thread's feature in every block
    const bool f_ok = fl < nfh;
    const int kb = 32 - __clz(B);                // bits of a bin in [0, B]
    // lanes of this lane's feature: those equal to it in the low log2(FS) bits
    unsigned long long flm = ~0ull;
    {
        constexpr unsigned long long kPat[6] = {0xAAAAAAAAAAAAAAAAull, 0xCCCCCCCCCCCCCCCCull, 0xF0F0F0F0F0F0F0F0ull,
                                                0xFF00FF00FF00FF00ull, 0xFFFF0000FFFF0000ull, 0xFFFFFFFF00000000ull};
#pragma unroll
        for (int i = 0; i < 6; ++i)
            if ((1 << i) < FS) flm &= ((fl >> i) & 1) ? kPat[i] : ~kPat[i];
    }
    const int n = s_nb[fl];
    const float *erow = s_edge + fl * (B + 1);   // edges k0 .. k0 + B
    const float *irow = s_iw + fl * B;           // inverse widths of bins k0 .. k0 + B - 1
    const unsigned long long lt = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
    // Each block's count row belongs to the one wave that ranks the block:
    // that wave zeroes the row first (its own stores stay in order, and the
    // previous sort's reads of the row finished before the caller's barrier).
    const int CS = cnt_stride(NK);
#pragma unroll
    for (int u = 0; u < kPR; ++u) {
        uint32_t *row = reinterpret_cast<uint32_t *>(s_cnt + ((tid + u * RB) >> 6) * CS);
        for (int i = lane; i < CS / 2; i += kWave) row[i] = 0u;
    }

    // A. keys and ranks: key | rank << 16 (keys below 2^16, ranks below 64)
#pragma unroll
    for (int u = 0; u < kPR; ++u) {
        const int p = tid + u * RB;
        const int s = p >> fs_shift;
        const int kg = clamp_bin(pk[u], n);     // the pair's bin; its place in the window:
        const bool inw = static_cast<unsigned>(kg - k0) < static_cast<unsigned>(B);
        const int k = inw ? kg - k0 : 0;
        const bool valid = f_ok && s < ns && inw;
        const float v = pv[u];
        const float e = erow[k];
        const uint32_t q = __float_as_uint(quant<Q>((v - e) * irow[k]));
        // x on e_k (k >= 1) gives q(frac) == +0 exactly; such rows carry -0
        // instead, which marks the edge term and adds the same zero
        qb[u] = (kg > 0 && v == e) ? 0x80000000u : (q == 0x80000000u ? 0u : q);
        const int kk = valid ? k : B;
        unsigned long long m = flm;
        for (int bit = 0; bit < kb; ++bit) {
            const bool set = (kk >> bit) & 1;
            const unsigned long long bal = __ballot(set);
            m &= set ? bal : ~bal;
        }
        const int rank = __popcll(m & lt);
        const int key = valid ? fl * B + k : NK;
        if (rank == 0 && key < NK) s_cnt[(p >> 6) * CS + key] = static_cast<uint16_t>(__popcll(m));
        ko[u] = key | (rank << 16);
    }
}

// kX: also x of every pair (xk, as ranked) to xs[sorted slot] (the linear0
// epilogue's per-row x).
template <int RB, bool kX = false>
__device__ __forceinline__ void tile_place(const BwdArgs &a, int tid, const int (&ko)[kP / RB],
                                           const uint32_t (&qb)[kP / RB], uint16_t *s_cnt, int *s_seg, int *s_tmp,
                                           uint2 *desc, uint32_t *piece, int *npc, const float (&xk)[kP / RB],
                                           float *xs) {
    constexpr int kPR = kP / RB;
    const int FS = a.FS, B = a.BW;
    const int fs_shift = __ffs(FS) - 1;
    const int NK = FS * B;
    const int lane = tid & (kWave - 1);
    const int wv = tid / kWave;
    const int fl = lane & (FS - 1);
    const int CS = cnt_stride(NK);

    // B. per key: block prefixes in place, then the scan over keys (rows in
    //    the low half, pieces in the high half; both below 2^16)
    const int kpt = (NK + RB - 1) / RB;
    const int j0 = min(NK, tid * kpt);
    const int j1 = min(NK, j0 + kpt);
    int local = 0;
    for (int j = j0; j < j1; ++j) {
        uint16_t *col = s_cnt + j;
        int cc[kBlocks];
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) cc[b] = col[b * CS];
        int run = 0;
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) {
            col[b * CS] = static_cast<uint16_t>(run);
            run += cc[b];
        }
        s_seg[j] = run;
        local += run | (((run + kL - 1) / kL) << 16);
    }
    int incl = local;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int v = __shfl_up(incl, o);
        if (lane >= o) incl += v;
    }
    if (lane == kWave - 1) s_tmp[wv] = incl;
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < RB / kWave; ++w) {
        const int tw = s_tmp[w];
        before += w < wv ? tw : 0;
        total += tw;
    }
    int run = before + incl - local;
    for (int j = j0; j < j1; ++j) {
        const int c = s_seg[j];
        s_seg[j] = run;
        run += c | (((c + kL - 1) / kL) << 16);
    }
    if (tid == 0) {
        s_seg[NK] = total;
        *npc = total >> 16;
    }
    __syncthreads();

    // C. scatter
#pragma unroll
    for (int u = 0; u < kPR; ++u) {
        const int key = ko[u] & 0xffff;
        if (key < NK) {
            const int p = tid + u * RB;
            const int s = p >> fs_shift;
            const int st = s_seg[key];
            const int within = s_cnt[(p >> 6) * CS + key] + (ko[u] >> 16);
            const int slot = (st & 0xffff) + within;
            desc[slot] = make_uint2(qb[u], static_cast<uint32_t>(s) | (static_cast<uint32_t>(fl) << 24));
            if constexpr (kX) xs[slot] = xk[u];
            if (within % kL == 0) {
                const int cnt = (s_seg[key + 1] & 0xffff) - (st & 0xffff);
                const int rows = min(kL, cnt - within);
                piece[(st >> 16) + within / kL] = static_cast<uint32_t>(key - fl * B) |
                                                  (static_cast<uint32_t>(fl) << 12) |
                                                  (static_cast<uint32_t>(slot) << 16) |
                                                  (static_cast<uint32_t>(rows - 1) << 28);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// reduce
// ---------------------------------------------------------------------------

template <int GD, int Q, int VEC, int LGW_T, int EPI, int RB>
__global__ __launch_bounds__(RB, 2) void ple_bwd_fused_kernel(BwdArgs a) {
    constexpr int NTH = RB;
    constexpr bool kRelu = (EPI & kBwdRelu) != 0;
    constexpr bool kLin = (EPI & kBwdLin) != 0;
    // A gradient that arrives in the quantisation dtype (or fp32 rounding)
    // is its own rounding: rounding it again changes nothing, and the bias
    // gradient is then the sum of the bin buckets (taken at finalize) -- also
    // linear0's bias gradient without a ReLU, whose buckets sum the unmasked
    // gradient.  Otherwise -- an fp32 gradient rounded to 16 bits, or linear0
    // behind a ReLU -- the bias gradient needs its own sum of the unrounded
    // (unmasked) gradient.  kFeatSums: per-feature sums in the records (that
    // one, and linear0's sum of g x).
    constexpr bool kGradExact = GD == Q || Q == PLE_DTYPE_F32;
    constexpr bool kRawDb = !kGradExact || (kLin && kRelu);
    constexpr bool kFeatSums = kRawDb || kLin;
    extern __shared__ __align__(16) unsigned char lds[];
    // B: the bins of a window (the LDS tables' and the keys' width); Bg: of the weight
    const int FS = a.FS, B = a.BW, D = a.D, F = a.F, NT = a.NT, Bg = a.B;
    float *s_qw = reinterpret_cast<float *>(lds + a.ro_qw);             // [FS][B+1][D] q(W) * iw, bins k0-1 ..
    float *s_hist = reinterpret_cast<float *>(lds + a.ro_hist);         // [FS][B][2D]
    float *s_db = reinterpret_cast<float *>(lds + a.ro_db);             // [FS][D]
    float *s_iw = reinterpret_cast<float *>(lds + a.ro_iw);             // [FS][B]
    int *s_nb = reinterpret_cast<int *>(lds + a.ro_nb);                 // [FS]
    // [P+2]: sorted rows, a dummy row, a discard slot.  Once a row's piece
    // is reduced, its dx replaces its q(frac) bits (.x), unless the dx are
    // staged in pair order (several features a group).
    uint2 *s_sdesc = reinterpret_cast<uint2 *>(lds + a.ro_desc);
    uint32_t *s_piece = reinterpret_cast<uint32_t *>(lds + a.ro_piece); // [PM]
    int *s_npc = reinterpret_cast<int *>(lds + a.ro_npc);               // [1]
    float *s_edge = reinterpret_cast<float *>(lds + a.ro_edge);         // [FS][B+1] (sort)
    uint16_t *s_cnt = reinterpret_cast<uint16_t *>(lds + a.ro_cnt);     // [P/64][cnt_stride(FS*B)] block counts (sort)
    int *s_seg = reinterpret_cast<int *>(lds + a.ro_seg);               // [FS*B+1] key starts (sort)
    int *s_tmp = reinterpret_cast<int *>(lds + a.ro_tmp);               // [RB/64] (sort)
    float *s_rec = reinterpret_cast<float *>(lds + a.ro_rec);           // [LG][RS]
    int *s_rkey = reinterpret_cast<int *>(lds + a.ro_rkey);             // [LG]
    int *s_rfl = reinterpret_cast<int *>(lds + a.ro_rfl);               // [LG] (kFeatSums)
    float *s_lw = reinterpret_cast<float *>(lds + a.ro_lw);             // [FS][D] linear0 weight
    float *s_dlw = reinterpret_cast<float *>(lds + a.ro_dlw);           // [FS][D] sum of g x
    float *s_xs = reinterpret_cast<float *>(lds + a.ro_xs);             // [P+1] x of the sorted rows (linear0)

    int g, c;
    if (!decode_tile(blockIdx.x, a.G, a.C, g, c)) return;
    // (the windows of a feature group are neighbours: they share its chunk's
    // bin indices and x in the L2)
    const int k0 = (g % a.NW) * B;   // the window's first bin
    g /= a.NW;
    const int f0 = g * FS;
    const int nfh = min(FS, F - f0);
    const int t_begin = c * a.SPC;
    const int t_end = min(a.T, t_begin + a.SPC);
    if (t_begin >= t_end) return;
    const int tid = threadIdx.x;
    const int PM = a.PM;

    // the sort's pairs of the next sub-tile (bin index, x), loaded a sub-tile
    // ahead
    int pk[kP / RB];
    float pv[kP / RB];
    auto load_pairs = [&](int t) __attribute__((always_inline)) {
        if (a.idxb == 1) tile_load<RB, uint8_t>(a, t, f0, nfh, tid, pk, pv);
        else if (a.idxb == 2) tile_load<RB, int16_t>(a, t, f0, nfh, tid, pk, pv);
        else tile_load<RB, int32_t>(a, t, f0, nfh, tid, pk, pv);
    };
    load_pairs(t_begin);
    int ko[kP / RB];          // the next sub-tile's keys | ranks, and q(frac) bits
    uint32_t qb[kP / RB];
    float xk[kP / RB];        // (linear0: their x)

    // ---- stage tables, clear accumulators ---------------------------------
    // Rows past a piece's end read the dummy row kP: q(frac) = +0 and sample
    // NT, whose gradient offset lies past every sub-tile's span (zeros).
    if (tid == 0) s_sdesc[kP] = make_uint2(0u, static_cast<uint32_t>(NT));
    if constexpr (kLin) {
        if (tid == 0) s_xs[kP] = 0.0f;   // (rows past a piece's end)
    }
    for (int i = tid; i < FS; i += NTH) s_nb[i] = i < nfh ? clamp_nbins(a.nbins[f0 + i], Bg) : 1;
    // (the window's inverse widths and edges; rows past the last feature are
    // never read: their pairs are padding)
    for (int i = tid; i < FS * B; i += NTH) {
        const int fl = i / B;
        const int kg = k0 + i - fl * B;
        s_iw[i] = fl < nfh && kg < Bg ? a.iw[static_cast<int64_t>(f0 + fl) * Bg + kg] : 0.0f;
    }
    for (int i = tid; i < FS * (B + 1); i += NTH) {
        const int fl = i / (B + 1);
        const int kg = k0 + i - fl * (B + 1);
        s_edge[i] = fl < nfh && kg <= Bg ? a.edges[static_cast<int64_t>(f0 + fl) * (Bg + 1) + kg] : 0.0f;
    }
    for (int i = tid; i < FS * B * 2 * D; i += NTH) s_hist[i] = 0.0f;
    for (int i = tid; i < FS * D; i += NTH) s_db[i] = 0.0f;
    if constexpr (kLin) {
        for (int i = tid; i < FS * D; i += NTH) {
            s_lw[i] = i / D < nfh ? a.lin_w[static_cast<int64_t>(f0) * D + i] : 0.0f;
            s_dlw[i] = 0.0f;
        }
    }
    __syncthreads();
    // the weight rows pre-scaled by their bin's inverse width: a row's dx term
    // iw_k <g, q(W[phys k])> is then one dot product with the table row.
    // Row r of a feature holds bin k0 + r - 1 (row 0: the bin below the
    // window, for the edge term of the window's first bin; zeros below bin 0).
    for (int i = tid; i < FS * (B + 1) * D; i += NTH) {
        const int fl = i / ((B + 1) * D);
        const int r = i - fl * ((B + 1) * D);
        const int rr = r / D;
        const int j = r - rr * D;
        const int kg = k0 + rr - 1;
        float w = 0.0f;
        if (fl < nfh) {
            const int n = s_nb[fl];
            if (kg >= 0 && kg < n) {
                const int64_t fr = static_cast<int64_t>(f0 + fl) * Bg;
                w = quant<Q>(a.weight[(fr + phys_bin(kg, n, Bg)) * D + j]) * a.iw[fr + kg];
            }
        }
        s_qw[i] = w;
    }

    // the first sub-tile's sort (the tables it reads are staged before the
    // barrier above), then the next sub-tile's pairs
    tile_rank<Q, RB>(a, t_begin, k0, nfh, tid, pk, pv, s_nb, s_edge, s_iw, s_cnt, ko, qb);
#pragma unroll
    for (int u = 0; u < kP / RB; ++u) xk[u] = kLin ? pv[u] : 0.0f;
    __syncthreads();
    tile_place<RB, kLin>(a, tid, ko, qb, s_cnt, s_seg, s_tmp, s_sdesc, s_piece, s_npc, xk, s_xs);
    if (t_begin + 1 < t_end) load_pairs(t_begin + 1);
    __syncthreads();

    const int lgw = LGW_T > 0 ? LGW_T : a.LGW;   // lanes per grad_output row (power of two)
    const int LG = RB / lgw;                  // lane groups (runs of pieces) per workgroup
    const int lg = tid / lgw;
    const int lc = tid - lg * lgw;
    const bool c_ok = lc < D / VEC;
    const int lcx = c_ok ? lc : 0;               // idle lanes read column 0 (their g is 0)
    const int D2 = 2 * D;
    // record stride {bucket | weighted (| raw g) (| g x)}
    const int RS = (kRawDb ? 3 * D : 2 * D) + (kLin ? D : 0);
    const int off_ax = D2 + (kRawDb ? D : 0);   // record offset of the g x sums (linear0)
    // dx of sorted row j: dword 2 j of the descriptors (row kP + 1 takes the
    // rows past a piece's end)
    uint32_t *s_dxw = reinterpret_cast<uint32_t *>(s_sdesc);
    // With several features a group the dx go through a staging buffer in
    // pair order (sample-major, s * FS + fl; slot kP discards) instead, so
    // that a sample's features leave in one store.
    const bool dx_staged = a.ro_dx >= 0;
    float *s_dx = reinterpret_cast<float *>(lds + (dx_staged ? a.ro_dx : 0));
    const int fs_shift = __ffs(FS) - 1;
    auto dx_slot = [&](uint32_t y) __attribute__((always_inline)) {
        return static_cast<int>(((y & 0xffffff) << fs_shift) + (y >> 24));
    };

    // F-phase state of a run: the key (feature, bin) of its first piece --
    // packed as fl << 12 | k, -1 for an empty run -- and that key's feature.
    // Each piece's sums go straight to LDS: those of the run's first key into
    // the run's record, every other key into the histogram (the run is that
    // key's only writer in this sub-tile), and likewise for the per-feature
    // sums.  Rows past a piece's end and idle lanes (lc >= D / VEC) load from
    // past the end of the gradient buffer, which reads zeros: they add
    // nothing and need no masking.
    int key0 = -1, fl0 = -1;
    float *rec = s_rec + lg * RS + lc * VEC;
    // Per-feature sums of the epilogue kernels (raw bias gradient, linear0's
    // g x) run in registers across the run's pieces and go to LDS when the
    // feature changes (rarely: a run spans at most FS features) and at the
    // run's end -- the first feature into the record, others into s_db /
    // s_dlw (this run is their only writer).
    int cur_fl = -1;
    float ad_run[VEC], ax_run[VEC];
#pragma unroll
    for (int q = 0; q < VEC; ++q) ad_run[q] = ax_run[q] = 0.0f;
    auto flush_feat = [&]() __attribute__((always_inline)) {
        if constexpr (kFeatSums) {
            if (cur_fl >= 0 && c_ok) {
                const bool first = cur_fl == fl0;
                if constexpr (kRawDb) {
                    float *dstd = first ? rec + D2 : s_db + __umul24(cur_fl, D) + lc * VEC;
                    float hd[VEC];
                    lds_load_vec<VEC>(dstd, hd);
#pragma unroll
                    for (int q = 0; q < VEC; ++q) hd[q] += ad_run[q];
                    lds_store_vec<VEC>(dstd, hd);
                }
                if constexpr (kLin) {
                    float *dstx = first ? rec + off_ax : s_dlw + __umul24(cur_fl, D) + lc * VEC;
                    float hx[VEC];
                    lds_load_vec<VEC>(dstx, hx);
#pragma unroll
                    for (int q = 0; q < VEC; ++q) hx[q] += ax_run[q];
                    lds_store_vec<VEC>(dstx, hx);
                }
            }
        }
    };

    // The current sub-tile: its descriptor and piece buffers, lane group
    // lg's run of contiguous pieces [j0, j1) (m pieces per run, the same for
    // every run), and its gradient rows as one buffer resource: byte offset
    // s * rowFb + fl * Db + lane offset (24-bit products: the planner keeps
    // the sub-tile's span below 2^31 bytes).  Offset `span` (first byte past
    // the sub-tile) stands in for rows past a piece's end and for idle lanes.
    constexpr uint32_t esz = GD == PLE_DTYPE_F32 ? 4 : 2;
    constexpr int kGW = grad_words<GD, VEC>();   // dwords of a row per lane (16-bit: two elements each)
    const uint32_t rowFb = static_cast<uint32_t>(F) * D * esz;
    const uint32_t Db = static_cast<uint32_t>(D) * esz;
    // Gradient rows of whole 128-byte lines are streamed (non-temporal
    // loads); other rows share lines with a neighbouring feature's rows,
    // which another run or workgroup reads later: narrower lane groups, the
    // rows of 2-float lanes (D = 2 mod 4), and the twins that the launcher
    // picks for rows of a lane group's width that end inside a line
    // (kBwdShared).  (Fixed per instantiation: a branch between the two
    // forms around the loads costs more than it saves.)
    constexpr int kGCpol =
        VEC % 4 == 0 && LGW_T * VEC * static_cast<int>(esz) >= 128 && (EPI & kBwdShared) == 0 ? kCpolNT : 0;
    // idle lanes: an offset past every span
    const uint32_t laneoff = c_ok ? static_cast<uint32_t>(lc) * VEC * esz : 0x80000000u;
    // ReLU input of a row (sample s, local feature fl): its mask word (the
    // one holding this lane's columns); rows past a piece's end (sample NT)
    // read zeros
    const int MW = a.MW;
    const uint32_t rowMb = static_cast<uint32_t>(F) * MW * 4;
    const uint32_t m_word_off = static_cast<uint32_t>((lcx * VEC) >> 5) * 4;
    const int m_shift = (lcx * VEC) & 31;
    // Lane groups of four or more lanes fetch a piece's ReLU mask words once
    // per quad of lanes: lane lc takes row lc & 3, then each row's word is
    // broadcast across the quad (DPP), instead of every lane loading all
    // four rows.  A quad's 4 * VEC columns lie in one mask word (VEC divides
    // 8), the word of the quad's first lane, which idle lanes take too.  (x of
    // a row, for linear0, comes with the sort: the ranked pairs' x go to LDS
    // in sorted order.)
    constexpr bool kQuadEpi = LGW_T >= 4;
    const int q_row = lc & 3;
    const uint32_t m_word_q =
        static_cast<uint32_t>(min(((lc & ~3) * VEC) >> 5, MW - 1)) * 4;
    const uint2 *t_desc = s_sdesc;
    const uint32_t *t_piece = s_piece;
    int64_t sub = 0;
    int ns = 0, m = 0, j0 = 0, j1 = 0;
    __amdgpu_buffer_rsrc_t grs = make_rsrc(a.g, 0u), mrs = grs;
    // sub-tile t, staged in LDS buffer b, becomes the current one
    auto set_tile = [&](int t, int b) __attribute__((always_inline)) {
        t_desc = s_sdesc + b * (kP + 1);
        t_piece = s_piece + b * PM;
        // (the same for every lane: kept in a scalar register, so the piece
        // loop's branches are scalar)
        const int NPc = __builtin_amdgcn_readfirstlane(s_npc[b]);
        m = (NPc + LG - 1) / LG;
        j0 = lg * m;
        j1 = min(j0 + m, NPc);
        key0 = j0 < j1 ? static_cast<int>(t_piece[j0] & 0xffff) : -1;
        fl0 = key0 >> 12;
        sub = static_cast<int64_t>(t) * NT;
        ns = static_cast<int>(min(static_cast<int64_t>(NT), a.N - sub));
        const int64_t row0 = sub * F + f0;
        grs = make_rsrc(static_cast<const char *>(a.g) + row0 * static_cast<int64_t>(D) * esz,
                        static_cast<uint32_t>(ns) * rowFb);
        if constexpr (kRelu) mrs = make_rsrc(a.mask + row0 * MW, static_cast<uint32_t>(ns) * F * MW * 4);
    };
    // Piece tt of the current sub-tile's run: its entry, its rows'
    // descriptors, and loads of their gradient rows.  Past j1 the piece is
    // empty (all rows read zeros).  Every lane loads, with no branch around the load,
    // so each piece has one counted wait.
    auto issue = [&](int tt, uint32_t (&gv)[kL][kGW], uint2 (&dv)[kL], uint32_t &pe, uint32_t (&mv)[kL],
                     float (&xv)[kL]) __attribute__((always_inline)) {
        const int j = j0 + tt;
        const bool real = j < j1;
        pe = t_piece[real ? j : 0];
        const int rs = static_cast<int>((pe >> 16) & 0xfff);
        const int n = real ? static_cast<int>(pe >> 28) + 1 : 0;
        const uint32_t flp = (pe >> 12) & 0xf;
        const uint32_t flb = __umul24(flp, Db) + laneoff;
#pragma unroll
        for (int i = 0; i < kL; ++i) dv[i] = t_desc[i < n ? rs + i : kP];
        // (the 24-bit products ignore the feature bits of .y)
#pragma unroll
        for (int i = 0; i < kL; ++i) load_grad_words<GD, VEC, kGCpol>(grs, __umul24(dv[i].y, rowFb) + flb, gv[i]);
        if constexpr (kQuadEpi && kRelu) {
            // this lane's row of the quad (selects on named values: indexing
            // the descriptor array would put it in scratch memory)
            const uint32_t y0 = dv[0].y, y1 = dv[1].y, y2 = dv[2].y, y3 = dv[3].y;
            const uint32_t yq = (q_row & 2) ? ((q_row & 1) ? y3 : y2) : ((q_row & 1) ? y1 : y0);
            if constexpr (kRelu)
                mv[0] = __builtin_amdgcn_raw_buffer_load_b32(
                    mrs, __umul24(yq, rowMb) + flp * static_cast<uint32_t>(MW) * 4 + m_word_q, 0, 0);
        } else {
            if constexpr (kRelu) {
#pragma unroll
                for (int i = 0; i < kL; ++i)
                    mv[i] = __builtin_amdgcn_raw_buffer_load_b32(
                        mrs, __umul24(dv[i].y, rowMb) + flp * static_cast<uint32_t>(MW) * 4 + m_word_off, 0, 0);
            }

        }
    };

    // Per piece: its key's row of the pre-scaled weight table (idle lanes
    // read column 0; their g is 0), the piece's sums in registers, then
    // added to LDS (the run's record or the histogram) before the next piece.
    // Row k-1 of the table serves rows with x on e_k (loaded only for them).
    auto process = [&](int tt, const uint32_t (&gv)[kL][kGW], const uint2 (&dsc)[kL], uint32_t pe,
                       const uint32_t (&mv)[kL], const float (&xv)[kL]) __attribute__((always_inline)) {
        const bool real = j0 + tt < j1;
        const int n = real ? static_cast<int>(pe >> 28) + 1 : 0;
        // (an empty piece past the run's end carries some piece's entry:
        // its table reads stay in range and it adds nothing)
        const int key = static_cast<int>(pe & 0xffff);
        const int fl = key >> 12;
        const int k = key & 0xfff;
        const int rowbase = __umul24(fl, B);
        // (table row of bin k: k + 1; of the bin below, for the edge term: k)
        const int qrow = __umul24(fl, B + 1) + k;
        float wk[VEC], lw[VEC], wp[VEC];
        lds_load_vec<VEC>(s_qw + __umul24(qrow + 1, D) + lcx * VEC, wk);
        if constexpr (kLin) lds_load_vec<VEC>(s_lw + __umul24(fl, D) + lcx * VEC, lw);
        float ab[VEC], aw[VEC];
        if constexpr (kFeatSums) {
            if (n > 0 && fl != cur_fl) {
                flush_feat();
                cur_fl = fl;
#pragma unroll
                for (int q = 0; q < VEC; ++q) ad_run[q] = ax_run[q] = 0.0f;
            }
        }
        // The piece's sums are added into LDS (a read-modify-write: this
        // lane group owns the cells): the run's first key (feature) into its
        // record, any other key (feature) into the histogram (bias sums).
        // The reads are issued here, ahead of the arithmetic; LDS keeps a
        // wave's accesses in order, so they see the previous piece's writes.
        // (Reads are harmless for idle lanes and empty pieces; only their
        // writes are skipped.)
        const bool add_ok = n > 0 && c_ok;
        float *dst = key == key0 ? rec : s_hist + __umul24(rowbase + k, D2) + lc * VEC;
        float hb[VEC], hw[VEC];
        lds_load_vec<VEC>(dst, hb);
        lds_load_vec<VEC>(dst + D, hw);
        // g of row i, column q of this lane: masked by the forward's ReLU
        // pass bit, rounded through Q
        auto g_masked = [&](int i, int q, uint32_t mvi) __attribute__((always_inline)) {
            float gm = grad_elem<GD>(gv[i], q);
            if constexpr (kRelu)
                gm = __uint_as_float(__float_as_uint(gm) &
                                     static_cast<uint32_t>(__builtin_amdgcn_sbfe(static_cast<int>(mvi), m_shift + q, 1)));
            return gm;
        };
        auto mask_word = [&](int i) __attribute__((always_inline)) -> uint32_t {
            if constexpr (kRelu) return kQuadEpi ? quad_bcast(mv[0], i) : mv[i];
            else return 0u;
        };
        // The edge term: a second pass over the registers that a wave takes
        // only when it holds an edge row, for the plain kernels; the module
        // epilogues' kernels fold it into the first pass (a second pass
        // there takes them past 256 VGPRs, one wave per SIMD).
        constexpr bool kEdgePass = !kRelu && !kLin;
        if constexpr (!kEdgePass) lds_load_vec<VEC>(s_qw + __umul24(qrow, D) + lcx * VEC, wp);
        float parts[kL];
        bool edge = false;
#pragma unroll
        for (int i = 0; i < kL; ++i) {
            const float qf = __uint_as_float(dsc[i].x);
            float dot = 0.0f, dotl = 0.0f, dot2 = 0.0f;
            const uint32_t mvi = mask_word(i);
            float xvi = 0.0f;
            if constexpr (kLin) xvi = s_xs[i < n ? ((pe >> 16) & 0xfff) + i : kP];
#pragma unroll
            for (int q = 0; q < VEC; ++q) {
                const float gm = g_masked(i, q, mvi);
                const float gq = kGradExact ? gm : quant<Q>(gm);
                // (the first row starts the piece's sums)
                ab[q] = i == 0 ? gq : ab[q] + gq;
                aw[q] = i == 0 ? qf * gq : fmaf(qf, gq, aw[q]);
                if constexpr (kRawDb) ad_run[q] += kLin ? grad_elem<GD>(gv[i], q) : gm;
                if constexpr (kLin) {
                    const float graw = grad_elem<GD>(gv[i], q);
                    ax_run[q] = fmaf(graw, xvi, ax_run[q]);
                    dotl = fmaf(graw, lw[q], dotl);
                }
                dot = fmaf(gq, wk[q], dot);
                if constexpr (!kEdgePass) dot2 = fmaf(gq, wp[q], dot2);
            }
            float part = dot;
            if constexpr (kLin) part += dotl;
            // x on the bin's left edge (k >= 1, marked by q(frac) = -0): the
            // lower bin's term too
            if constexpr (!kEdgePass) part = dsc[i].x == 0x80000000u ? part + dot2 : part;
            parts[i] = part;
            edge = edge || dsc[i].x == 0x80000000u;
        }
        // Edge rows are rare in most data: the wave takes this branch only
        // when one of its lane groups holds one.
        if (kEdgePass && __any(edge)) {
            lds_load_vec<VEC>(s_qw + __umul24(qrow, D) + lcx * VEC, wp);
#pragma unroll
            for (int i = 0; i < kL; ++i) {
                const uint32_t mvi = mask_word(i);
                float dot2 = 0.0f;
#pragma unroll
                for (int q = 0; q < VEC; ++q) {
                    const float gm = g_masked(i, q, mvi);
                    dot2 = fmaf(kGradExact ? gm : quant<Q>(gm), wp[q], dot2);
                }
                if (dsc[i].x == 0x80000000u) parts[i] += dot2;
            }
        }
        if (add_ok) {
#pragma unroll
            for (int q = 0; q < VEC; ++q) {
                hb[q] += ab[q];
                hw[q] += aw[q];
            }
            lds_store_vec<VEC>(dst, hb);
            lds_store_vec<VEC>(dst + D, hw);
        }
        // dx into the rows' descriptors (rows past the piece's end: the
        // discard slot)
        const int rs = static_cast<int>((pe >> 16) & 0xfff);
        if constexpr (LGW_T >= 4) {
            // reduce-scatter: each lane ends with one row's sum (32- and
            // 64-lane groups: within each 16-lane row, then across the rows)
            static_assert(kL == 4, "four rows per piece");
            constexpr int kW = LGW_T >= 32 ? 16 : LGW_T;
            constexpr int kLog = kW == 4 ? 2 : (kW == 8 ? 3 : 4);
            const int r = (((lc >> (kLog - 1)) & 1) << 1) | ((lc >> (kLog - 2)) & 1);
            float v = group_reduce_scatter4<kW>(parts, lc & (kW - 1));
            if constexpr (LGW_T >= 32) v += __shfl_xor(v, 16);
            if constexpr (LGW_T == 64) v += __shfl_xor(v, 32);
            if (dx_staged) {
                // (selects on named values: indexing the descriptor array
                // with r would put it in scratch memory)
                const uint32_t y0 = dsc[0].y, y1 = dsc[1].y, y2 = dsc[2].y, y3 = dsc[3].y;
                const uint32_t yr = (r & 2) ? ((r & 1) ? y3 : y2) : ((r & 1) ? y1 : y0);
                s_dx[r < n ? dx_slot(yr) : kP] = v;
            } else {
                s_dxw[2 * (r < n ? rs + r : kP + 1)] = __float_as_uint(v);
            }
        } else {
#pragma unroll
            for (int i = 0; i < kL; ++i) {
                float v = parts[i];
                if constexpr (LGW_T > 0) v = group_sum<LGW_T>(v);
                else v = group_sum_rt(v, lgw);
                if (dx_staged) s_dx[i < n ? dx_slot(dsc[i].y) : kP] = v;
                else s_dxw[2 * (i < n ? rs + i : kP + 1)] = __float_as_uint(v);
            }
        }
    };

    // Three register buffers: pieces tt+1 and tt+2 are in flight while piece
    // tt is reduced (enough bytes in flight for one workgroup to keep its
    // CU's share of HBM busy while the other one sorts).  m is the same for
    // every run, so the loop is uniform; a piece issued past a run's end is
    // empty.  A sub-tile's first two pieces are issued as soon as its
    // descriptors are in place.
    uint32_t gA[kL][kGW], gB[kL][kGW], gC[kL][kGW];
    uint2 dA[kL], dB[kL], dC[kL];
    uint32_t pA = 0, pB = 0, pC = 0;
    uint32_t mA[kL], mB[kL], mC[kL];     // (epilogue with ReLU)
    float xA[kL], xB[kL], xC[kL];        // (epilogue with linear0)
    auto begin_tile = [&](int t) __attribute__((always_inline)) {
        set_tile(t, 0);
        if (m > 0) {
            issue(0, gA, dA, pA, mA, xA);
            issue(1, gB, dB, pB, mB, xB);
        }
    };


    // Per sub-tile t (its first pieces in flight): the ranking part of sub-tile
    // t + 1's sort, then F reduces t's pieces; after a barrier H and G store
    // its dx and merge its run records, and the placing part of the sort
    // fills the descriptor buffer for t + 1; after another barrier its first
    // pieces are issued.
    begin_tile(t_begin);
    for (int t = t_begin; t < t_end; ++t) {
        const bool more = t + 1 < t_end;
        if (more) {
            tile_rank<Q, RB>(a, t + 1, k0, nfh, tid, pk, pv, s_nb, s_edge, s_iw, s_cnt, ko, qb);
            if constexpr (kLin) {
#pragma unroll
                for (int u = 0; u < kP / RB; ++u) xk[u] = pv[u];
            }
            if (t + 2 < t_end) load_pairs(t + 2);
        }

        // F. pieces: lane group lg takes the contiguous pieces [j0, j1) (its
        //    "run"); piece 0 is in flight already
        // the run's record starts at zero (its reads by the previous
        // sub-tile's merge finished before the sort's barriers)
        if (c_ok) {
            float z[VEC];
#pragma unroll
            for (int q = 0; q < VEC; ++q) z[q] = 0.0f;
            for (int h = 0; h < RS; h += D) lds_store_vec<VEC>(rec + h, z);
        }
        if (lc == 0) {
            s_rkey[lg] = key0;
            if constexpr (kFeatSums) s_rfl[lg] = fl0;
        }
        cur_fl = -1;
        if (m > 0) {
            int tt = 0;
#pragma unroll 1
            for (; tt + 2 < m; tt += 3) {
                issue(tt + 2, gC, dC, pC, mC, xC);
                process(tt, gA, dA, pA, mA, xA);
                issue(tt + 3, gA, dA, pA, mA, xA);   // (unconditional: one block per step schedules better)
                process(tt + 1, gB, dB, pB, mB, xB);
                issue(tt + 4, gB, dB, pB, mB, xB);
                process(tt + 2, gC, dC, pC, mC, xC);
            }
            if (tt < m) process(tt, gA, dA, pA, mA, xA);
            if (tt + 1 < m) process(tt + 1, gB, dB, pB, mB, xB);
        }
        flush_feat();
        __syncthreads();
        const int64_t h_sub = sub;
        const int h_ns = ns;

        // H. dx of the sub-tile's rows (one per valid pair: ns * nfh), from
        //    the staging buffer or the descriptors straight into dx [N, F].
        //    The lines of a sample's features fill up in the L2 of the XCD,
        //    which runs every feature group of the chunk (decode_tile).
        if (a.dx && dx_staged) {
#pragma unroll
            for (int u = 0; u < (kP / RB); ++u) {
                const int p = tid + u * RB;
                const int sidx = p >> fs_shift;
                const int fl = p & (FS - 1);
                if (fl < nfh && sidx < h_ns) a.dx[(h_sub + sidx) * F + f0 + fl] = s_dx[p];
            }
        } else if (a.dx) {
            // (the sub-tile's sorted rows: its pairs in this window)
            const int rows = s_seg[FS * B] & 0xffff;
#pragma unroll
            for (int u = 0; u < (kP / RB); ++u) {
                const int j = tid + u * RB;
                if (j < rows) {
                    const uint2 d = s_sdesc[j];
                    a.dx[(h_sub + (d.y & 0xffffff)) * F + f0 + (d.y >> 24)] = __uint_as_float(d.x);
                }
            }
        }

        // G. run records, one run of equal keys (features) per head, in order
        if (c_ok) {
            const int key = s_rkey[lg];
            if (key >= 0 && (lg == 0 || s_rkey[lg - 1] != key)) {
                float sb[VEC], sw[VEC];
#pragma unroll
                for (int q = 0; q < VEC; ++q) sb[q] = sw[q] = 0.0f;
                for (int j = lg; j < LG && s_rkey[j] == key; ++j) {
                    const float *rj = s_rec + j * RS + lc * VEC;
#pragma unroll
                    for (int q = 0; q < VEC; ++q) {
                        sb[q] += rj[q];
                        sw[q] += rj[D + q];
                    }
                }
                float *h = s_hist + (static_cast<size_t>(key >> 12) * B + (key & 0xfff)) * D2 + lc * VEC;
#pragma unroll
                for (int q = 0; q < VEC; ++q) {
                    h[q] += sb[q];
                    h[D + q] += sw[q];
                }
            }
            const int rfl = kFeatSums ? s_rfl[lg] : -1;
            if (kFeatSums && rfl >= 0 && (lg == 0 || s_rfl[lg - 1] != rfl)) {
                float sd[VEC], sx[VEC];
#pragma unroll
                for (int q = 0; q < VEC; ++q) sd[q] = sx[q] = 0.0f;
                for (int j = lg; j < LG && s_rfl[j] == rfl; ++j) {
                    const float *rj = s_rec + j * RS + lc * VEC;
#pragma unroll
                    for (int q = 0; q < VEC; ++q) {
                        if constexpr (kRawDb) sd[q] += rj[D2 + q];
                        if constexpr (kLin) sx[q] += rj[off_ax + q];
                    }
                }
#pragma unroll
                for (int q = 0; q < VEC; ++q) {
                    if constexpr (kRawDb) s_db[rfl * D + lc * VEC + q] += sd[q];
                    if constexpr (kLin) s_dlw[rfl * D + lc * VEC + q] += sx[q];
                }
            }
        }
        // S. the placing part of the next sub-tile's sort (its first barrier
        //    also orders the record reads above before the next sub-tile's
        //    record writes)
        if (more) tile_place<RB, kLin>(a, tid, ko, qb, s_cnt, s_seg, s_tmp, s_sdesc, s_piece, s_npc, xk, s_xs);
        // this barrier orders the histogram updates before the next
        // sub-tile's pieces, the sort's descriptors before they are read, and
        // the count reads before the next ranking zeroes them
        __syncthreads();
        if (more) begin_tile(t + 1);
    }
    __syncthreads();

    // One chunk: this workgroup has seen every sample of its features, so it
    // writes dW and db from the LDS histogram itself, with the finalize
    // kernel's steps and lane count (dw_suffix; the results repeat those of
    // the two-kernel path bitwise), kFinLanes lanes per column, columns in
    // turn.  Whole lane groups run every pass (a group past the live columns
    // scans zeros).
    if (a.fin_fused) {
        constexpr int kGroups = NTH / kFinLanes;
        const int l = tid % kFinLanes;
        const int D2 = 2 * D;
        for (int col0 = 0; col0 < nfh * D; col0 += kGroups) {
            const int col = col0 + tid / kFinLanes;
            const bool ok = col < nfh * D;
            const int fl = ok ? col / D : 0;
            const int j = ok ? col - fl * D : 0;
            const int n = ok ? s_nb[fl] : 0;
            // (one window: B == Bg)
            const float *h = s_hist + static_cast<size_t>(fl) * B * D2 + j;   // bucket at k * D2, weighted at + D
            auto total = [&](int k, int hh) __attribute__((always_inline)) { return h[k * D2 + hh * D]; };
            float *dwc = ok && a.dw ? a.dw + static_cast<int64_t>(f0 + fl) * Bg * D + j : nullptr;
            const float incl = dw_suffix(total, n, Bg, D, l, dwc);
            if (ok && l == 0) {
                const int64_t fj = static_cast<int64_t>(f0 + fl) * D + j;
                if (a.db) a.db[fj] = a.db_from_buckets ? incl : s_db[fl * D + j];
                if constexpr (kLin) {
                    if (a.dlw) a.dlw[fj] = s_dlw[fl * D + j];
                }
            }
        }
        return;
    }

    // chunk partials
    if (a.part) {
        // (the window's cells: bins k0 .. k0 + B - 1 of the partials' Bg)
        const int D2 = 2 * D;
        float *dst = a.part + (static_cast<int64_t>(c) * F + f0) * Bg * D2 + static_cast<int64_t>(k0) * D2;
        for (int i = tid; i < FS * B * D2; i += NTH) {
            const int fl = i / (B * D2);
            const int r = i - fl * B * D2;
            if (fl < nfh && k0 + r / D2 < s_nb[fl]) dst[static_cast<int64_t>(fl) * Bg * D2 + r] = s_hist[i];
        }
        if constexpr (kRawDb) {
            float *dstb = a.part_db + (static_cast<int64_t>(c) * F + f0) * D;
            for (int i = tid; i < FS * D; i += NTH)
                if (i / D < nfh) dstb[i] = s_db[i];
        }
        if constexpr (kLin) {
            float *dstl = a.part_lw + (static_cast<int64_t>(c) * F + f0) * D;
            for (int i = tid; i < FS * D; i += NTH)
                if (i / D < nfh) dstl[i] = s_dlw[i];
        }
    }
}

// ---------------------------------------------------------------------------
// 16-bit gradients on the matrix cores
// ---------------------------------------------------------------------------

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short v8s_t __attribute__((ext_vector_type(8)));
typedef short v4s_t __attribute__((ext_vector_type(4)));

// gfx950's transposing LDS read: within each group of 16 lanes, lane r
// addresses 4 consecutive 16-bit elements (a row of a 16 x 4 block, 8-byte
// aligned) and lane j receives element j % 4 of rows j / 4, j / 4 + 4,
// j / 4 + 8, j / 4 + 12 (the mapping checked on an MI355X).  With lane r
// addressing sample s0 + r / 4, columns 4 (r % 4) .. of a row-major block,
// lane j receives column j of samples s0 .. s0 + 3.
__device__ __forceinline__ v4s_t lds_read_tr16(const short *p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4s_t *)(const_cast<short *>(p)));
}

// C += A B on a 32x32x16 matrix instruction, 16-bit operands, fp32
// accumulation: A 32 x 16, lane l holding A[l % 32][8 (l / 32) + t] in its
// element t (t = 0..7); B 16 x 32, lane l holding B[8 (l / 32) + t][l % 32];
// C 32 x 32, lane l's register r holding C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]
// (the layout checked on an MI355X against a host product, bf16 and fp16).
// The eight 16-bit elements of an operand come packed in four dwords,
// element t in bits 16 (t % 2) of dword t / 2.
template <int GD>
__device__ __forceinline__ f32x16_t mfma16(uint4 a, uint4 b, f32x16_t c) {
    if constexpr (GD == PLE_DTYPE_BF16) {
        typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0,
                                                        0, 0);
    } else {
        typedef _Float16 v8h __attribute__((ext_vector_type(8)));
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0,
                                                       0);
    }
}

// Two 16-bit lanes at once.  min and negation are asm (the compiler turns the
// equivalent vector code back into compares and selects); the multiply-add
// that feeds the matrix instruction stays compiler code, so the compiler sees
// the VALU write of that operand and keeps the wait states a matrix
// instruction needs after it (an asm producer is invisible to that check)
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// c + a.lo * b.lo + a.hi * b.hi, 16-bit pairs (bf16 or fp16), fp32 sum
template <int GD>
__device__ __forceinline__ float dot2_16(uint32_t a, uint32_t b, float c) {
    if constexpr (GD == PLE_DTYPE_BF16) {
        typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a), __builtin_bit_cast(bf2, b), c, false);
    } else {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
    }
}
__device__ __forceinline__ uint32_t pk_min_u16(uint32_t a, uint32_t b) {
    uint32_t r;
    __asm__("v_pk_min_u16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ uint32_t pk_neg_u16(uint32_t a) {
    uint32_t r;
    __asm__("v_pk_sub_u16 %0, 0, %1" : "=v"(r) : "v"(a));
    return r;
}
__device__ __forceinline__ uint32_t pk_mad_u16(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) * __builtin_bit_cast(u16x2, b) +
                                            __builtin_bit_cast(u16x2, c));
}

constexpr int kMB = 32;                            // samples per block (the products' K: two steps of 16)
constexpr int kMfmaWaves = 8;                      // waves per workgroup
constexpr int kMfmaBlock = kMfmaWaves * kWave;
constexpr int kMfmaPF = 1;                         // steps whose loads are in flight (1 or 2)
constexpr int kBPW = 2;                            // blocks of a wave in a step (worked on together)
// blocks whose dx a wave stores together (c4, the whole kernel: 8 -> 211,
// 16 -> 216, 32 -> 223, 4 -> 228 us)
constexpr int kDxB = 8;
// a staged row: 36 16-bit columns (72 bytes: the 8-byte reads of 32
// consecutive rows meet distinct banks; columns D..35 stay zero, the
// products' columns past D); a feature's rows of a step, then 32 bytes
// that put the next feature's rows on other banks
constexpr int kRowCols = 36;
constexpr int kRowBytes = 2 * kRowCols;
constexpr int kStepSamples = kMfmaWaves * kBPW * kMB;   // samples x features a step
constexpr int kAreaPad = 48;   // the next feature's rows 12 banks on
constexpr size_t kStageRows = static_cast<size_t>(kStepSamples) * kRowBytes + 4 * kAreaPad;
// bytes of one stage: the rows, x [256 / FS][FS], the bin-index words (or
// bytes)
constexpr size_t kStageBytes = kStageRows + 4 * kStepSamples + 4 * kStepSamples;
// per wave, not staged: the block's bins and q(frac) bits, 16-bit, [64]
// each (lanes 32..63 write copies to the upper half), the dx of kDxB blocks
constexpr int kMfmaWaveBytes = kBPW * (2 * 64 + 2 * 64) + 4 * kMB * kDxB;
// non-finite gradient values a workgroup records (with a count and, per
// feature of the group, a mask of the columns whose records overflowed)
constexpr int kMfmaEvents = 512;
constexpr size_t kMfmaEvBytes = 32 + 8 * kMfmaEvents;
constexpr int kMfmaMaxBins = 96;   // three tiles of 32 bins
// table loads a thread has in flight in the set-up (c4, the whole kernel:
// 4 / 8 -> 203-204 us, 16 -> 209-211, 32 -> 213-215)
constexpr int kTabLoads = 8;
constexpr int kMfmaFinLanes = 4;   // lanes of a (feature, column) in the kernel's dW / db step
// the set-up reads a group's iw and edges one entry a thread, and clears the
// stages 16 bytes at a time
static_assert(4 * (kMfmaMaxBins + 1) <= kMfmaBlock, "iw / edge tables: one entry a thread");
static_assert(kStageBytes % 16 == 0, "stages cleared in 16-byte stores");

// A gradient already in the 16-bit quantisation dtype (bf16 or fp16) makes
// every factor of the histograms exact in that dtype: bin k's bucket sum is
// onehot_k^T g and its weighted sum (onehot_k * q(frac))^T g over the
// samples, so the histograms of a block of 32 samples are two products of
// the (bins x samples) one-hot matrices with the block's (samples x columns)
// gradient, fp32-accumulated by the matrix instruction in an order it fixes:
// deterministic, and no sort.
//
// One workgroup per (group of FS adjacent features, chunk of samples), in
// steps of 512 / FS samples.  The workgroup loads a step together -- the FS
// rows of a sample are contiguous, so the loads cover whole runs of memory
// (rows of 48 bytes read one feature at a time, each at its sample's stride,
// draw about half the rate) -- into LDS, two stages deep: the rows feature
// by feature, x, and the words holding the bin indices.  Wave w takes
// feature w % FS and blocks 2 (w / FS) and 2 (w / FS) + 1 of each step (two
// blocks side by side hide each other's LDS round trips), and keeps that
// feature's histograms (NBT tiles of 32 bins, bucket and weighted) in its
// accumulators.  Lane l holds sample l % 32 of a block, the half l / 32 of
// its row (4 NQ columns): its bin, q(frac) and dx come out of registers --
// dx as iw_k times the half row's dot product with q(W[k]) (plus iw_{k-1}
// times the one with q(W[k-1]) for x on a left edge), the two halves added
// low half first.  At the end the waves of a feature add their histograms in
// LDS in wave order, and they go, like the sorted path's, to dW / db (one
// chunk) or to the chunk partials.  Rows of D = 8 NQ columns (NQ = 1..4), at
// most 32 NBT bins; bin indices are uint8.
template <int GD, int NBT, int NQ>
__global__ __launch_bounds__(kMfmaBlock, 1) void ple_bwd_mfma_kernel(BwdArgs a) {
    constexpr int D = 8 * NQ;
    constexpr int D2 = 2 * D;
    constexpr int DH = 4 * NQ;   // columns of a half row
    constexpr uint32_t kOne = GD == PLE_DTYPE_BF16 ? 0x3F80u : 0x3C00u;   // 1.0
    extern __shared__ __align__(16) unsigned char lds[];
    const int B = a.B, F = a.F, FS = a.FS;
    const int WPF = kMfmaWaves / FS;   // waves a feature
    const int SPS = kMB * kBPW * WPF;  // samples a step
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int fl = wave % FS;   // the wave's feature in the group
    const int wf = wave / FS;   // and its block in a step

    int fg, c;
    if (!decode_tile(blockIdx.x, a.G, a.C, fg, c)) return;
    const int64_t n_begin = static_cast<int64_t>(c) * a.NC;
    const int64_t n_end = min(a.N, n_begin + a.NC);
    if (n_begin >= n_end) return;
    const int f0 = fg * FS;
    const int f = f0 + fl;
    const bool fok = f < F;
    const int n = fok ? clamp_nbins(a.nbins[f], B) : 1;   // the wave's feature's bins
    // the group's tables: [FS][B+1][D] q(W) in the 16-bit dtype (exact; row
    // r: bin r - 1), [FS][B] iw, [FS][B+1] edges; then the two stages and the
    // waves' areas, which the histograms [FS][B][2D] take over after the stream
    const uint16_t *s_qh = reinterpret_cast<const uint16_t *>(lds + a.ro_qw) + fl * (B + 1) * D;
    float *s_iw = reinterpret_cast<float *>(lds + a.ro_iw) + fl * B;
    float *s_edge = reinterpret_cast<float *>(lds + a.ro_edge) + fl * (B + 1);
    float *s_hist = reinterpret_cast<float *>(lds + a.ro_hist);
    unsigned char *s_stage = lds + a.ro_desc;
    unsigned char *wb = lds + a.ro_desc + 2 * kStageBytes + wave * kMfmaWaveBytes;
    uint32_t *s_evn = reinterpret_cast<uint32_t *>(lds + a.ro_tmp);   // [0] records, [4 + fl] overflow columns
    uint2 *s_ev = reinterpret_cast<uint2 *>(lds + a.ro_tmp + 32);     // {bin | col << 8 | fl << 16, g | q << 16}
    uint16_t *s_bin = reinterpret_cast<uint16_t *>(wb);                 // [kBPW][64] bin, 0xffff past the batch
    uint16_t *s_q = reinterpret_cast<uint16_t *>(wb + kBPW * 128);      // [kBPW][64] q(frac) bits
    float *s_dxb = reinterpret_cast<float *>(wb + kBPW * 256);          // [kDxB][32] dx
    const int area = SPS * kRowBytes + kAreaPad;   // bytes of a feature's rows in a stage
    auto st_rows = [&](int buf, int ff) { return s_stage + buf * kStageBytes + ff * area; };
    auto st_x = [&](int buf) { return reinterpret_cast<float *>(s_stage + buf * kStageBytes + kStageRows); };
    auto st_k = [&](int buf) {
        return reinterpret_cast<uint32_t *>(s_stage + buf * kStageBytes + kStageRows + 4 * kStepSamples);
    };

    // ---- the loads of a step: kBPW NQ 8-byte pieces a lane in address order -
    // piece u = tid + kMfmaBlock r of the step's SPS x FS D / 4 pieces:
    // sample u / CPS, feature (u % CPS) / (D / 4), columns 4 (u % (D / 4)) ..
    const int CPS = FS * D / 4;   // pieces a sample
    const uint32_t rowFb = static_cast<uint32_t>(F) * D * 2;
    const int gspan = min(FS, F - f0) * D * 2;   // bytes of the group's row that exist
    constexpr int NP = kBPW * NQ;   // pieces a lane
    uint32_t poff[NP];              // the piece's byte offset in the step's rows
    int prow[NP];                   // its place in a stage
    bool pok[NP];                   // its feature exists
#pragma unroll
    for (int r = 0; r < NP; ++r) {
        const int u = tid + kMfmaBlock * r;
        const int s = u / CPS, q = u - s * CPS;
        const int ff = q / (D / 4), cq = q - ff * (D / 4);
        poff[r] = static_cast<uint32_t>(s) * rowFb + static_cast<uint32_t>(q) * 8;
        prow[r] = ff * area + s * kRowBytes + cq * 8;
        pok[r] = f0 + ff < F;
    }
    // x and the bin indices: lane t < SPS FS takes x of (sample t / FS,
    // feature t % FS) and the aligned 32-bit word holding its bin byte (a
    // whole word, in the page of the byte: every load of the stream is then
    // one instruction of one width, so the compiler's waits for a step's
    // loads leave the later steps' loads in flight)
    uint2 gq[kMfmaPF][NP];
    float px[kMfmaPF];
    uint32_t pk[kMfmaPF];
    const int nsteps = static_cast<int>((n_end - n_begin + SPS - 1) / SPS);
    auto load_step = [&](int p, int st) __attribute__((always_inline)) {
        const int64_t s0 = n_begin + static_cast<int64_t>(st) * SPS;
        const int ns = st < nsteps ? static_cast<int>(min(static_cast<int64_t>(SPS), n_end - s0)) : 0;
        const __amdgpu_buffer_rsrc_t rs =
            make_rsrc(static_cast<const char *>(a.g) + (s0 * F + f0) * static_cast<int64_t>(D) * 2,
                      ns > 0 ? static_cast<uint32_t>(ns - 1) * rowFb + static_cast<uint32_t>(gspan) : 0u);
#pragma unroll
        for (int r = 0; r < NP; ++r) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, poff[r], 0, 0);
            gq[p][r] = make_uint2(v[0], v[1]);
        }
        const int xs = tid / FS, xf = tid - xs * FS;
        const bool xok = tid < SPS * FS && xs < ns && f0 + xf < F;
        const int64_t pair = xok ? (s0 + xs) * F + f0 + xf : 0;
        px[p] = a.x[pair];
        const uint8_t *kb8 = static_cast<const uint8_t *>(a.idx) + pair;
        pk[p] = *reinterpret_cast<const uint32_t *>(kb8 - (reinterpret_cast<uintptr_t>(kb8) & 3));
    };
    // the first step's loads go out before the tables' (the stream's first
    // wait overlaps the set-up)
#pragma unroll
    for (int p = 0; p < kMfmaPF; ++p) load_step(p, p);

    // ---- tables; the transposed blocks' columns past D stay zero ----------
    // Every load of the set-up is unconditional (an entry that does not exist
    // reads entry 0 and is replaced by zero) and issued in rounds of kTabLoads
    // before the round's first use: the set-up waits for the memory a few
    // times, not once or twice per entry.
    int nfe[4];   // the group's features' bin counts (0 past F)
#pragma unroll
    for (int ff = 0; ff < 4; ++ff) nfe[ff] = ff < FS && f0 + ff < F ? clamp_nbins(a.nbins[f0 + ff], B) : 0;
    auto nbins_of = [&](int ff) __attribute__((always_inline)) {
        return ff == 0 ? nfe[0] : ff == 1 ? nfe[1] : ff == 2 ? nfe[2] : nfe[3];
    };
    {
        // iw and edges: FS (B + 1) <= 4 * 97 entries, one a thread
        const bool iok = tid < FS * B && f0 + tid / B < F;
        const bool eok = tid < FS * (B + 1) && f0 + tid / (B + 1) < F;
        const float iv = a.iw[iok ? static_cast<int64_t>(f0) * B + tid : 0];
        const float ev = a.edges[eok ? static_cast<int64_t>(f0) * (B + 1) + tid : 0];
        const int ntab = FS * (B + 1) * D;
        for (int i0 = 0; i0 < ntab; i0 += kTabLoads * kMfmaBlock) {
            float wv[kTabLoads];
            bool wok[kTabLoads];
#pragma unroll
            for (int u = 0; u < kTabLoads; ++u) {
                const int i = i0 + u * kMfmaBlock + tid;
                const int ff = i / ((B + 1) * D);
                const int rem = i - ff * (B + 1) * D;
                const int rr = rem / D;
                const int j = rem - rr * D;
                const int kg = rr - 1;
                const int na = nbins_of(ff);
                wok[u] = i < ntab && kg >= 0 && kg < na;
                wv[u] = a.weight[wok[u] ? ((static_cast<int64_t>(f0 + ff) * B + phys_bin(kg, na, B)) * D + j) : 0];
            }
#pragma unroll
            for (int u = 0; u < kTabLoads; ++u) {
                const int i = i0 + u * kMfmaBlock + tid;
                const uint16_t w = !wok[u] ? 0
                                   : GD == PLE_DTYPE_BF16 ? static_cast<uint16_t>(__float_as_uint(quant<GD>(wv[u])) >> 16)
                                                          : f16_bits(wv[u]);
                if (i < ntab) reinterpret_cast<uint16_t *>(lds + a.ro_qw)[i] = w;
            }
        }
        if (tid < FS * B) reinterpret_cast<float *>(lds + a.ro_iw)[tid] = iok ? iv : 0.0f;
        if (tid < FS * (B + 1)) reinterpret_cast<float *>(lds + a.ro_edge)[tid] = eok ? ev : 0.0f;
    }
    for (int i = tid; i < static_cast<int>(2 * kStageBytes / 16); i += kMfmaBlock)
        reinterpret_cast<uint4 *>(s_stage)[i] = make_uint4(0u, 0u, 0u, 0u);
    if (tid < 8) s_evn[tid] = 0u;
    __syncthreads();

    // a step's loads into LDS stage buf: the rows, feature by feature, x,
    // the index words (or bytes)
    auto stage_step = [&](int p, int buf) __attribute__((always_inline)) {
        unsigned char *rows = st_rows(buf, 0);
#pragma unroll
        for (int r = 0; r < NP; ++r)
            *reinterpret_cast<uint2 *>(rows + prow[r]) = pok[r] ? gq[p][r] : make_uint2(0u, 0u);
        if (tid < SPS * FS) {
            st_x(buf)[tid] = px[p];
            st_k(buf)[tid] = pk[p];
        }
    };

    // ---- the wave's block of each step --------------------------------------
    const int sl = lane % 32;   // the lane's sample in a block
    const int h = lane / 32;    // and its half row: columns DH h .. DH h + DH - 1
    // the transposing reads of the products' B operand: lane l of group
    // l / 16 addresses sample 8 h + (l % 16) / 4 (+ 4 for the second read),
    // columns 16 ((l / 16) % 2) + 4 (l % 4) .. of the block's staged rows
    const int tr_off = (8 * h + (lane % 16) / 4) * kRowCols + 16 * ((lane / 16) % 2) + 4 * (lane % 4);
    f32x16_t hb[NBT], hw[NBT];
#pragma unroll
    for (int T = 0; T < NBT; ++T)
#pragma unroll
        for (int r = 0; r < 16; ++r) hb[T][r] = hw[T][r] = 0.0f;
    // the one-hot operands, two samples a dword: per 16-bit half,
    // m = min(bin ^ lane's bin, 1) is 0 on a hit, and m * (-v) + v gives v on
    // a hit, 0 otherwise (v = 1.0 for the bucket sums, q(frac) for the
    // weighted ones)
    uint32_t lbin[NBT];
#pragma unroll
    for (int T = 0; T < NBT; ++T) lbin[T] = static_cast<uint32_t>(32 * T + sl) * 0x10001u;
    const uint32_t one2 = kOne * 0x10001u;
    const uint32_t negone2 = (0x10000u - kOne) * 0x10001u;
    const uint32_t ones = 0x10001u;
    // dx of the wave's last kDxB blocks, stored together and waited for at
    // once: no store is left in flight among the loads (with one, the
    // compiler's next wait for a load would cover every load in flight)
    int nbuf = 0, buf_first = 0;
    auto flush_dx = [&]() __attribute__((always_inline)) {
        if (a.dx) {
            for (int e = lane; e < nbuf * kBPW * kMB; e += kWave) {
                const int bi = e / kMB;
                const int64_t s = n_begin + static_cast<int64_t>(buf_first + bi / kBPW) * SPS +
                                  (kBPW * wf + bi % kBPW) * kMB + (e - bi * kMB);
                if (s < n_end) a.dx[s * F + f] = s_dxb[e];
            }
            __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        }
    };
    auto blocks = [&](int st, int buf) __attribute__((always_inline)) {
        // the lane's sample of each block: bin, q(frac), left edge (x on e_k,
        // k >= 1); the blocks' steps side by side
        int k[kBPW];
        bool valid[kBPW], edge[kBPW];
        float qf[kBPW], dot[kBPW], iwk[kBPW];
        uint2 gv[kBPW][NQ];
        const unsigned char *rows[kBPW];
#pragma unroll
        for (int i = 0; i < kBPW; ++i) {
            const int sb0 = (kBPW * wf + i) * kMB;   // the block's first sample in the step
            valid[i] = n_begin + static_cast<int64_t>(st) * SPS + sb0 + sl < n_end;
            const int64_t pr = valid[i] ? (n_begin + static_cast<int64_t>(st) * SPS + sb0 + sl) * F + f : 0;
            const int kshift = 8 * static_cast<int>((reinterpret_cast<uintptr_t>(a.idx) + pr) & 3);
            const uint32_t kw = st_k(buf)[(sb0 + sl) * FS + fl];
            k[i] = clamp_bin(static_cast<int>((kw >> kshift) & 0xffu), n);
            const float xv = st_x(buf)[(sb0 + sl) * FS + fl];
            const float e = s_edge[k[i]];
            iwk[i] = s_iw[k[i]];
            qf[i] = quant<GD>((xv - e) * iwk[i]);
            edge[i] = k[i] > 0 && xv == e;
            // the lane's half row
            rows[i] = st_rows(buf, fl) + sb0 * kRowBytes;
            const unsigned char *row = rows[i] + sl * kRowBytes + h * DH * 2;
#pragma unroll
            for (int j = 0; j < NQ; ++j) gv[i][j] = *reinterpret_cast<const uint2 *>(row + 8 * j);
            // dx: iw_k times the half row's dot product with q(W[k]) (pairs of
            // 16-bit products, exact, summed in fp32)
            const uint16_t *wr = s_qh + (k[i] + 1) * D + DH * h;
            float d = 0.0f;
#pragma unroll
            for (int j = 0; j < NQ; ++j) {
                const uint2 wv = *reinterpret_cast<const uint2 *>(wr + 4 * j);
                d = dot2_16<GD>(gv[i][j].x, wv.x, d);
                d = dot2_16<GD>(gv[i][j].y, wv.y, d);
            }
            dot[i] = d * iwk[i];
        }
        // and iw_{k-1} times the one with q(W[k-1]) on a left edge, in a pass
        // taken when the wave holds one
        if (__ballot(edge[0] || edge[kBPW - 1])) {
#pragma unroll
            for (int i = 0; i < kBPW; ++i) {
                const int km = k[i] > 0 ? k[i] - 1 : 0;
                const uint16_t *wr = s_qh + k[i] * D + DH * h;
                float d2 = 0.0f;
#pragma unroll
                for (int j = 0; j < NQ; ++j) {
                    const uint2 wv = *reinterpret_cast<const uint2 *>(wr + 4 * j);
                    d2 = dot2_16<GD>(gv[i][j].x, wv.x, d2);
                    d2 = dot2_16<GD>(gv[i][j].y, wv.y, d2);
                }
                if (edge[i]) dot[i] += d2 * s_iw[km];
            }
        }
        // Non-finite gradient values: in the products, 0 * inf would spread
        // them to every bin of their column; they leave the block (zeros in
        // its staged rows) and are added to their own bin's cells at the end,
        // as the sorted path sums them.  A half row holding one has a
        // non-finite dot product (inf times a weight is +-inf or NaN).
        if (__ballot((valid[0] && !__builtin_isfinite(dot[0])) ||
                     (valid[kBPW - 1] && !__builtin_isfinite(dot[kBPW - 1])))) {
#pragma unroll
            for (int i = 0; i < kBPW; ++i) {
                if (!valid[i] || __builtin_isfinite(dot[i])) continue;
                uint16_t *hr = reinterpret_cast<uint16_t *>(const_cast<unsigned char *>(rows[i]) + sl * kRowBytes +
                                                            h * DH * 2);
                const uint32_t qbits = GD == PLE_DTYPE_BF16 ? (__float_as_uint(qf[i]) >> 16) : f16_bits(qf[i]);
                for (int e = 0; e < DH; ++e) {
                    const uint32_t gb = hr[e];
                    const uint32_t em = GD == PLE_DTYPE_BF16 ? 0x7F80u : 0x7C00u;   // exponent bits
                    if ((gb & em) != em) continue;
                    const int col = DH * h + e;
                    const uint32_t slot = atomicAdd(&s_evn[0], 1u);
                    if (slot < static_cast<uint32_t>(kMfmaEvents))
                        s_ev[slot] = make_uint2(static_cast<uint32_t>(k[i]) | (col << 8) | (fl << 16), gb | (qbits << 16));
                    else
                        atomicOr(&s_evn[4 + fl], 1u << col);
                    hr[e] = 0;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < kBPW; ++i) {
            // the two halves' sums, low half first, in every lane: gfx950's
            // v_permlane32_swap (a VALU exchange of the wave's halves, no LDS
            // round trip) gives lane l the value of lane l % 32 and of lane
            // l % 32 + 32 (the mapping checked on an MI355X)
            const uint32_t db = __float_as_uint(dot[i]);
            const auto halves = __builtin_amdgcn_permlane32_swap(db, db, false, false);
            s_dxb[(nbuf * kBPW + i) * kMB + sl] = __uint_as_float(halves[0]) + __uint_as_float(halves[1]);
            s_bin[i * 64 + lane] = static_cast<uint16_t>(valid[i] ? k[i] : 0xffff);
            s_q[i * 64 + lane] =
                GD == PLE_DTYPE_BF16 ? static_cast<uint16_t>(__float_as_uint(qf[i]) >> 16) : f16_bits(qf[i]);
        }
        // the histograms: two steps of 16 samples a block; A = the one-hot
        // (and q-weighted one-hot) rows of this lane's bins, B = the gradient:
        // column sl of samples sb .. sb + 7 (zero past D), by two transposing
        // LDS reads of 4 samples each
#pragma unroll
        for (int i = 0; i < kBPW; ++i) {
            const short *gtr = reinterpret_cast<const short *>(rows[i]) + tr_off;
#pragma unroll
            for (int ks = 0; ks < kMB / 16; ++ks) {
                const int sb = 16 * ks + 8 * h;
                const v4s_t lo = lds_read_tr16(gtr + 16 * ks * kRowCols);
                const v4s_t hi = lds_read_tr16(gtr + (16 * ks + 4) * kRowCols);
                const v8s_t bv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                const uint4 bop = __builtin_bit_cast(uint4, bv);
                const uint4 kb = *reinterpret_cast<const uint4 *>(s_bin + i * 64 + sb);
                const uint4 qb = *reinterpret_cast<const uint4 *>(s_q + i * 64 + sb);
                const uint32_t kv[4] = {kb.x, kb.y, kb.z, kb.w};
                const uint32_t qv[4] = {qb.x, qb.y, qb.z, qb.w};
                uint32_t nq[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) nq[j] = pk_neg_u16(qv[j]);
#pragma unroll
                for (int T = 0; T < NBT; ++T) {
                    uint32_t ab[4], aw[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t m = pk_min_u16(kv[j] ^ lbin[T], ones);
                        ab[j] = pk_mad_u16(m, negone2, one2);
                        aw[j] = pk_mad_u16(m, nq[j], qv[j]);
                    }
                    hb[T] = mfma16<GD>(make_uint4(ab[0], ab[1], ab[2], ab[3]), bop, hb[T]);
                    hw[T] = mfma16<GD>(make_uint4(aw[0], aw[1], aw[2], aw[3]), bop, hw[T]);
                }
            }
        }
        if (++nbuf == kDxB / kBPW) {
            flush_dx();
            nbuf = 0;
            buf_first = st + 1;
        }
    };

    // ---- steps: stage, refill, barrier, blocks ------------------------------
    // (stage buf is rewritten two steps later, after the next step's barrier:
    // every wave has left this step's blocks by then)
    const bool mine = fok;
    int st = 0;
    for (; st + 1 < nsteps; st += 2) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            stage_step(p % kMfmaPF, p);
            load_step(p % kMfmaPF, st + p + kMfmaPF);
            __syncthreads();
            if (mine && n_begin + static_cast<int64_t>(st + p) * SPS + kBPW * wf * kMB < n_end) blocks(st + p, p);
        }
    }
    if (st < nsteps) {
        stage_step(0, 0);
        __syncthreads();
        if (mine && n_begin + static_cast<int64_t>(st) * SPS + kBPW * wf * kMB < n_end) blocks(st, 0);
    }
    if (mine) flush_dx();
    __syncthreads();

    // ---- the feature's waves add their histograms in LDS, in wave order -----
    float *hf = s_hist + fl * B * D2;
    for (int w = 0; w < WPF; ++w) {
        if (wf == w && fok && sl < D) {
#pragma unroll
            for (int T = 0; T < NBT; ++T)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int i = 32 * T + 8 * (r / 4) + 4 * h + r % 4;
                    if (i < B) {
                        float *hp = hf + i * D2;
                        if (w == 0) {
                            hp[sl] = hb[T][r];
                            hp[D + sl] = hw[T][r];
                        } else {
                            hp[sl] += hb[T][r];
                            hp[D + sl] += hw[T][r];
                        }
                    }
                }
        }
        __syncthreads();
    }

    // the recorded non-finite values into their bins' cells, in record order
    // (inf and NaN sums do not depend on it); columns whose records
    // overflowed become NaN
    if (tid == 0 && (s_evn[0] | s_evn[4] | s_evn[5] | s_evn[6] | s_evn[7]) != 0u) {
        const int ne = min(static_cast<int>(s_evn[0]), kMfmaEvents);
        for (int e = 0; e < ne; ++e) {
            const uint2 r = s_ev[e];
            const int bin = r.x & 0xff, col = (r.x >> 8) & 0xff, ff = r.x >> 16;
            const float g = GD == PLE_DTYPE_BF16 ? __uint_as_float((r.y & 0xffffu) << 16)
                                                 : f16_to_float(static_cast<uint16_t>(r.y));
            const float q = GD == PLE_DTYPE_BF16 ? __uint_as_float(r.y & 0xffff0000u)
                                                 : f16_to_float(static_cast<uint16_t>(r.y >> 16));
            float *hp = s_hist + (ff * B + bin) * D2;
            hp[col] += g;
            hp[D + col] += q * g;
        }
        for (int ff = 0; ff < FS; ++ff)
            for (int col = 0; col < D; ++col)
                if (s_evn[4 + ff] >> col & 1u)
                    for (int bin = 0; bin < B; ++bin)
                        s_hist[(ff * B + bin) * D2 + col] = s_hist[(ff * B + bin) * D2 + D + col] = __builtin_nanf("");
    }
    __syncthreads();

    if (a.fin_fused) {
        // one chunk: dW and db from the histograms (the finalize kernel's
        // steps), one (feature, column) per kMfmaFinLanes lanes: the FS D <=
        // 128 columns of the group in one round
        constexpr int kGroups = kMfmaBlock / kMfmaFinLanes;
        const int l = tid % kMfmaFinLanes;
        for (int p0 = 0; p0 < FS * D; p0 += kGroups) {
            const int pr = p0 + tid / kMfmaFinLanes;
            const int ff = pr / D;
            const int fa = f0 + ff;
            const bool ok = pr < FS * D && fa < F;
            const int j = ok ? pr - ff * D : 0;
            const int nn = ok ? nbins_of(ff) : 0;
            const float *hp = s_hist + (ok ? ff : 0) * B * D2 + j;
            auto total = [&](int k, int hh) __attribute__((always_inline)) { return hp[k * D2 + hh * D]; };
            float *dwc = ok && a.dw ? a.dw + static_cast<int64_t>(fa) * B * D + j : nullptr;
            const float incl = dw_suffix<kMfmaFinLanes>(total, nn, B, D, l, dwc);
            if (ok && l == 0 && a.db) a.db[static_cast<int64_t>(fa) * D + j] = incl;
        }
        return;
    }
    if (a.part) {
        for (int ff = 0; ff < FS && f0 + ff < F; ++ff) {
            const int nn = nbins_of(ff);
            float *dst = a.part + (static_cast<int64_t>(c) * F + f0 + ff) * B * D2;
            for (int i = tid; i < nn * D2; i += kMfmaBlock) dst[i] = s_hist[ff * B * D2 + i];
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
        float s = 0.0f, s2 = 0.0f, sl = 0.0f;
        for (int j = gl; j < D; j += kLanes) {
            const float graw = load_grad<GD>(a.g, p * D + j);
            float gm = graw;
            if (a.mask && !((a.mask[p * a.MW + (j >> 5)] >> (j & 31)) & 1u)) gm = 0.0f;
            const float gv = quant<Q>(gm);
            s = fmaf(gv, quant<Q>(w[j]), s);
            if (edge) s2 = fmaf(gv, quant<Q>(wp[j]), s2);
            if (a.lin_w) sl = fmaf(graw, a.lin_w[static_cast<int64_t>(f) * D + j], sl);
        }
#pragma unroll
        for (int off = kLanes / 2; off > 0; off >>= 1) {
            s += __shfl_xor(s, off, kLanes);
            s2 += __shfl_xor(s2, off, kLanes);
            sl += __shfl_xor(sl, off, kLanes);
        }
        if (gl == 0) {
            float r = s * a.iw[static_cast<int64_t>(f) * B + k];
            if (edge) r = fmaf(s2, a.iw[static_cast<int64_t>(f) * B + k - 1], r);
            if (a.lin_w) r += sl;
            a.dx[p] = r;
        }
    }
}

// One wave per (feature, sample chunk, block of 64 columns); lane jj owns
// column j = 64 * block + jj and walks the chunk in sample order, folding
// runs of equal bins into its own cells: in LDS ({bucket} [B][W] then
// {weighted} [B][W], W = the block's columns), copied to the chunk's partials
// at the end, or -- GLOBAL, tables beyond LDS -- straight in the chunk's
// partials [B][2D] in global memory, which only this lane reads and writes.
// Either way one fixed order per cell.
template <int GD, int Q, typename IdxT, bool GLOBAL>
__global__ __launch_bounds__(kWave) void ple_bwd_simple_hist_kernel(BwdArgs a) {
    extern __shared__ float smem[];
    const int B = a.B, D = a.D, F = a.F;
    const int f = blockIdx.x % F;
    const int c = (blockIdx.x / F) % a.C;
    const int jb = blockIdx.x / (F * a.C) * kWave;     // the block's first column
    const int W = min(kWave, D - jb);                  // its columns
    const int jj = threadIdx.x;
    const int j = jb + jj;
    const bool jok = jj < W;
    const int n_real = clamp_nbins(a.nbins[f], B);
    float *dst = a.part + (static_cast<int64_t>(c) * F + f) * B * 2 * D;
    // bucket / weighted cell of bin k for this lane's column
    float *hb = GLOBAL ? dst + j : smem + jj;
    float *hw = GLOBAL ? dst + D + j : smem + static_cast<int64_t>(B) * W + jj;
    const int cstride = GLOBAL ? 2 * D : W;
    if (jok) {
        for (int k = 0; k < n_real; ++k) {
            hb[static_cast<int64_t>(k) * cstride] = 0.0f;
            hw[static_cast<int64_t>(k) * cstride] = 0.0f;
        }
    }
    if constexpr (!GLOBAL) __syncthreads();
    const int64_t n_begin = static_cast<int64_t>(c) * a.NC;
    const int64_t n_end = min(a.N, n_begin + a.NC);
    const float *e = a.edges + static_cast<int64_t>(f) * (B + 1);
    const float *iwr = a.iw + static_cast<int64_t>(f) * B;
    int kc = -1;
    float cb = 0.0f, cw = 0.0f, cdb = 0.0f, clw = 0.0f;
    constexpr int kBatch = 16;
    for (int64_t n0 = n_begin; n0 < n_end; n0 += kBatch) {
        int kk[kBatch];
        float xv[kBatch];
        float gv[kBatch];
        uint32_t mv[kBatch];
#pragma unroll
        for (int t = 0; t < kBatch; ++t) {
            const int64_t n = n0 + t;
            const bool ok = n < n_end;
            const int64_t p = n * F + f;
            kk[t] = ok ? clamp_bin(load_idx<IdxT>(a.idx, p), n_real) : 0;
            xv[t] = ok ? a.x[p] : 0.0f;
            gv[t] = (ok && jok) ? load_grad<GD>(a.g, p * D + j) : 0.0f;
            mv[t] = (ok && jok && a.mask) ? a.mask[p * a.MW + (j >> 5)] : ~0u;
        }
#pragma unroll
        for (int t = 0; t < kBatch; ++t) {
            if (n0 + t >= n_end) break;
            const int k = kk[t];
            const float qf = quant<Q>((xv[t] - e[k]) * iwr[k]);
            const float graw = gv[t];
            // ReLU epilogue: the forward's pass bit; linear0 sums use the raw g
            const float gm = ((mv[t] >> (j & 31)) & 1u) ? graw : 0.0f;
            const float gq = quant<Q>(gm);
            if (a.lin_w) clw = fmaf(graw, xv[t], clw);
            if (k != kc) {
                if (kc >= 0 && jok) {
                    hb[static_cast<int64_t>(kc) * cstride] += cb;
                    hw[static_cast<int64_t>(kc) * cstride] += cw;
                }
                kc = k;
                cb = gq;
                cw = qf * gq;
            } else {
                cb += gq;
                cw = fmaf(qf, gq, cw);
            }
            cdb += a.lin_w ? graw : gm;
        }
    }
    if (kc >= 0 && jok) {
        hb[static_cast<int64_t>(kc) * cstride] += cb;
        hw[static_cast<int64_t>(kc) * cstride] += cw;
    }
    if constexpr (!GLOBAL) {
        __syncthreads();
        for (int i = jj; i < n_real * W; i += kWave) {
            const int k = i / W;
            const int col = jb + (i - k * W);
            dst[static_cast<int64_t>(k) * 2 * D + col] = smem[i];
            dst[static_cast<int64_t>(k) * 2 * D + D + col] = smem[static_cast<int64_t>(B) * W + i];
        }
    }
    if (jok) a.part_db[(static_cast<int64_t>(c) * F + f) * D + j] = cdb;
    if (jok && a.lin_w) a.part_lw[(static_cast<int64_t>(c) * F + f) * D + j] = clw;
}

// ---------------------------------------------------------------------------
// chunk sums: the partials of every chunk added, in chunk order, into chunk 0
// ---------------------------------------------------------------------------

// Partials [Cd][per-chunk elements]; one thread per element of chunk 0, its
// Cd loads issued eight at a time.  Each element is read and rewritten by one
// thread only, so the sum lands in place.
__global__ __launch_bounds__(kBlock) void ple_bwd_chunksum_kernel(float *part, int64_t per_chunk, int Cd) {
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; e < per_chunk;
         e += static_cast<int64_t>(gridDim.x) * kBlock) {
        float *base = part + e;
        float s = 0.0f;
        int cc = 0;
        for (; cc + 8 <= Cd; cc += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = base[(cc + u) * per_chunk];
#pragma unroll
            for (int u = 0; u < 8; ++u) s += v[u];
        }
        for (; cc < Cd; ++cc) s += base[cc * per_chunk];
        base[0] = s;
    }
}

// ---------------------------------------------------------------------------
// finalize: one workgroup per (feature, group of kFinCols columns)
// ---------------------------------------------------------------------------


// Sums the chunk partials of every (bin, column) of the group in chunk order
// into LDS (or reads their sums from chunk 0, where ple_bwd_chunksum_kernel
// left them: many bins or chunks), then kFinLanes lanes per column take the
// suffix over logical bins (dw_suffix).  The bias gradient is the sum of all
// buckets (fp32 gradients) or its own summed partials.  A fixed order
// throughout: results repeat bitwise.

__global__ __launch_bounds__(kBlock) void ple_bwd_finalize_kernel(BwdArgs a) {
    extern __shared__ float tot[];       // [n][2][kFinStride]
    const int f = blockIdx.x;
    const int j0 = blockIdx.y * kFinCols;
    const int B = a.B, D = a.D;
    const int D2 = 2 * D;
    const int nc = min(kFinCols, D - j0);
    const int n = clamp_nbins(a.nbins[f], B);
    const int tid = threadIdx.x;
    const float *src = a.part + static_cast<int64_t>(f) * B * D2;
    const bool need_tot = !a.fin_direct && (a.dw || (a.db && a.db_from_buckets));
    const int col = tid / kFinLanes;
    const int l = tid % kFinLanes;
    // bin k's chunk sum of half h (0: bucket, 1: weighted) for this lane's column
    // (fin_direct implies summed chunks)
    auto total = [&](int k, int h) {
        if (!a.fin_direct) return tot[(k * 2 + h) * kFinStride + col];
        return src[k * D2 + h * D + j0 + col];
    };
    const int nsum = a.fin_summed ? 1 : a.Cd;
    const int64_t cstride = static_cast<int64_t>(a.F) * B * D2;
    if (need_tot) {
        // element e -> (bin k, half h: bucket / weighted, column j0 + c); a
        // thread's kFinBatch elements load together, four chunks at a time
        // (each element still summed in chunk order), so the loads of a
        // batch wait for the memory once per four chunks, not once per load
        const int ne = n * 2 * kFinCols;
        for (int e0 = 0; e0 < ne; e0 += kFinBatch * kBlock) {
            const float *pe[kFinBatch];
            bool ok[kFinBatch];
            float sum[kFinBatch];
#pragma unroll
            for (int u = 0; u < kFinBatch; ++u) {
                const int e = e0 + u * kBlock + tid;
                const int k = e / (2 * kFinCols);
                const int h = (e / kFinCols) & 1;
                const int cidx = e % kFinCols;
                ok[u] = e < ne && cidx < nc;
                pe[u] = src + (ok[u] ? k * D2 + h * D + j0 + cidx : 0);   // (else a valid address, ignored)
                sum[u] = 0.0f;
            }
            int cc = 0;
            for (; cc + 4 <= nsum; cc += 4) {
                float v[4][kFinBatch];
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int u = 0; u < kFinBatch; ++u) v[t][u] = pe[u][(cc + t) * cstride];
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int u = 0; u < kFinBatch; ++u) sum[u] += v[t][u];
            }
            for (; cc < nsum; ++cc) {
                float v[kFinBatch];
#pragma unroll
                for (int u = 0; u < kFinBatch; ++u) v[u] = pe[u][cc * cstride];
#pragma unroll
                for (int u = 0; u < kFinBatch; ++u) sum[u] += v[u];
            }
#pragma unroll
            for (int u = 0; u < kFinBatch; ++u) {
                const int e = e0 + u * kBlock + tid;
                if (e < ne) tot[(e / kFinCols) * kFinStride + e % kFinCols] = ok[u] ? sum[u] : 0.0f;
            }
        }
        __syncthreads();
    }
    if (col >= nc) return;   // (whole half-waves: the scan below stays within live lanes)
    const int j = j0 + col;
    const int64_t wrow = static_cast<int64_t>(f) * B;
    const bool sum_buckets = a.dw || (a.db && a.db_from_buckets);
    if (sum_buckets) {
        const float incl = dw_suffix(total, n, B, D, l, a.dw ? a.dw + wrow * D + j : nullptr);
        if (a.db && a.db_from_buckets && l == 0) a.db[static_cast<int64_t>(f) * D + j] = incl;
    }
    if (l == 0) {
        const int64_t fj = static_cast<int64_t>(f) * D + j;
        const int64_t dstride = static_cast<int64_t>(a.F) * D;
        if (a.db && !a.db_from_buckets) {
            float sb = 0.0f;
            for (int cc = 0; cc < a.Cd; ++cc) sb += a.part_db[cc * dstride + fj];
            a.db[fj] = sb;
        }
        if (a.dlw) {
            float sl = 0.0f;
            for (int cc = 0; cc < a.Cd; ++cc) sl += a.part_lw[cc * dstride + fj];
            a.dlw[fj] = sl;
        }
    }
}

// ---------------------------------------------------------------------------
// planning
// ---------------------------------------------------------------------------

constexpr size_t kPartialBudget = 64ull << 20;   // bytes of chunk partials
// LDS per reduce workgroup the planner aims for: two workgroups per CU (the
// kernel's registers allow two waves per SIMD)
constexpr size_t kReduceLdsTarget = 80 * 1024;

struct BwdPlan {
    bool sorted;
    int mfma_nbt = 0;   // > 0: ple_bwd_mfma_kernel with this many 32-bin tiles
    int mfma_nq = 0;    // and rows of 8 mfma_nq columns
    bool hist_global;   // fallback: histogram cells in global memory (tables beyond LDS)
    int vec;
    int rb;          // reduce workgroup size
    int C, Cd;
    int64_t NC;
    size_t lds;
    size_t part_bytes, part_db_bytes, part_lw_bytes;
    BwdArgs geo;     // sorted-path geometry and LDS offsets
    size_t total() const {
        return align_up(part_bytes, 256) + align_up(part_db_bytes, 256) + align_up(part_lw_bytes, 256);
    }
};

struct LdsTaker {
    size_t off = 0;
    void operator()(int &field, size_t bytes) {
        field = static_cast<int>(off);
        off = align_up(off + bytes, 16);
    }
};

// B: the bins of a window.  raw_db: records carry the raw-gradient bias sums
// too (quantised gradients, linear0 epilogue); lin: and the linear0 weight
// sums.  The sort's edges, block counts, key starts and wave totals.
size_t reduce_layout(BwdArgs &g, int FS, int B, int D, int LG, int PM, bool raw_db, bool lin) {
    constexpr int bufs = 1;
    const int NK = FS * B;
    LdsTaker take;
    take(g.ro_qw, 4ull * FS * (B + 1) * D);
    take(g.ro_hist, 8ull * FS * B * D);
    take(g.ro_db, 4ull * FS * D);
    take(g.ro_iw, 4ull * FS * B);
    take(g.ro_nb, 4ull * FS);
    take(g.ro_desc, bufs * 8ull * (kP + 2));
    take(g.ro_piece, bufs * 4ull * PM);
    take(g.ro_npc, bufs * 4ull);
    take(g.ro_rec, (8ull + (raw_db ? 4ull : 0ull) + (lin ? 4ull : 0ull)) * LG * D);
    take(g.ro_rkey, 4ull * LG);
    take(g.ro_rfl, raw_db || lin ? 4ull * LG : 0ull);
    take(g.ro_dx, FS > 1 ? 4ull * (kP + 1) : 0ull);
    take(g.ro_lw, lin ? 4ull * FS * D : 0ull);
    take(g.ro_dlw, lin ? 4ull * FS * D : 0ull);
    take(g.ro_xs, lin ? 4ull * (kP + 1) : 0ull);
    take(g.ro_edge, 4ull * FS * (B + 1));
    take(g.ro_cnt, 2ull * kBlocks * cnt_stride(NK));
    take(g.ro_seg, 4ull * (NK + 1));
    take(g.ro_tmp, 4ull * (kWideBlock / kWave));
    if (FS == 1) g.ro_dx = -1;
    return take.off;
}

// LDS of the matrix-core kernel: the FS features' tables, then the two
// stages and the waves' areas, which the histograms take over after the
// stream, then the non-finite records
size_t mfma_layout(BwdArgs &g, int B, int D, int FS) {
    LdsTaker take;
    take(g.ro_qw, 2ull * FS * (B + 1) * D);
    take(g.ro_iw, 4ull * FS * B);
    take(g.ro_edge, 4ull * FS * (B + 1));
    take(g.ro_desc, std::max<size_t>(2 * kStageBytes + static_cast<size_t>(kMfmaWaves) * kMfmaWaveBytes,
                                     8ull * FS * B * D));
    g.ro_hist = g.ro_desc;
    take(g.ro_tmp, kMfmaEvBytes);
    return take.off;
}

// g_align16: the gradient's base address is 16-byte aligned; g16: the
// gradient is a 16-bit type; raw_db: the bias gradient needs its own sums
// (an fp32 gradient rounded to 16 bits, or linear0); lin: linear0 sums
BwdPlan plan_backward(int64_t N, int64_t F, int64_t B, int64_t D, bool g_align16, bool g16, bool raw_db, bool lin) {
    BwdPlan pl{};
    pl.rb = kBlock;
    const int cus = device_cu_count();
    pl.sorted = false;
    // A 16-bit gradient that is its own rounding (raw_db false for a 16-bit
    // gradient: its quantisation dtype is its own), rows of 8, 16, 24 or 32
    // columns, at most 96 bins (three tiles: the accumulators of four leave
    // too few registers), a step's rows within 32-bit offsets: the
    // matrix-core kernel, one workgroup per (group of FS features, chunk):
    // FS = 4 adjacent features where LDS holds their tables (2, 1 else),
    // chunks for a workgroup per CU (its eight waves fill the CU's two waves
    // per SIMD) within the partials budget -- where that takes at most 8
    // chunks: with more, shorter chunks' set-up, histogram merge and partials
    // cost more than the sorted path (knob PLE_TUNE_BWD_MFMA: 1 never, 2
    // whenever the shape allows).
    const int mfma_knob = tuning(PLE_TUNE_BWD_MFMA);
    if (g16 && !raw_db && !lin && g_align16 && D % 8 == 0 && D <= 32 && B <= kMfmaMaxBins &&
        static_cast<int64_t>(kStepSamples) * F * D * 2 < INT32_MAX && mfma_knob != 1 &&
        tuning(PLE_TUNE_BWD_SIMPLE) == 0) {
        BwdArgs geo{};
        int fs = 4;
        while (fs > 1 && (fs > F || mfma_layout(geo, static_cast<int>(B), static_cast<int>(D), fs) > kLdsMax))
            fs /= 2;
        if (tuning(PLE_TUNE_BWD_FS) == 1 || tuning(PLE_TUNE_BWD_FS) == 2 || tuning(PLE_TUNE_BWD_FS) == 4)
            fs = std::min<int>(tuning(PLE_TUNE_BWD_FS), fs);
        geo.FS = fs;
        geo.G = static_cast<int>((F + fs - 1) / fs);
        const int64_t per_chunk = F * B * 2 * D * 4;
        int64_t c = (static_cast<int64_t>(cus) + geo.G - 1) / geo.G;
        const int64_t budget_c = static_cast<int64_t>(kPartialBudget) / per_chunk;
        if (c > budget_c) c = budget_c;
        // a few steps for every chunk
        const int64_t max_c = N / (static_cast<int64_t>(kMB) * 4 * (kMfmaWaves / fs));
        if (c > max_c) c = max_c;
        if (c < 1) c = 1;
        if (c <= 8 || mfma_knob == 2) {
            pl.mfma_nbt = static_cast<int>((B + 31) / 32);
            pl.mfma_nq = static_cast<int>(D / 8);
            pl.rb = kMfmaBlock;
            pl.vec = 4;
            int64_t nc = (N + c - 1) / c;
            nc = (nc + kMB - 1) / kMB * kMB;
            pl.NC = nc;
            pl.lds = mfma_layout(geo, static_cast<int>(B), static_cast<int>(D), fs);
            pl.C = pl.Cd = static_cast<int>((N + nc - 1) / nc);
            pl.geo = geo;
            if (pl.C > 1) {
                pl.part_bytes = static_cast<size_t>(pl.Cd) * F * B * 2 * D * sizeof(float);
                pl.part_db_bytes = static_cast<size_t>(pl.Cd) * F * D * sizeof(float);
            }
            return pl;
        }
    }
    // Sorted path: a sub-tile's gradient rows span less than 2^31 bytes
    // (32-bit buffer offsets); the bins of a workgroup fit the 12-bit field of
    // a piece -- all of them, or a window of them.
    if (static_cast<int64_t>(kP) * F * D * 4 < INT32_MAX && tuning(PLE_TUNE_BWD_SIMPLE) == 0) {
        // 4 floats per lane (16-byte loads for fp32 gradients) when D allows
        // (8 a lane halved the per-row instructions but needed registers for
        // two waves per SIMD only, and hid less latency); lane groups of a
        // power-of-two width
        int vec = !g_align16 ? 1 : (D % 4 == 0 ? 4 : 1);
        // even D not a multiple of 4 (up to 64 columns): 2 floats per lane,
        // half the loads of one per lane and lane groups with DPP sums
        if (vec == 1 && g_align16 && D % 2 == 0 && D >= 6 && D <= 64) vec = 2;
        // 16-bit gradients: 8 elements (one 16-byte load) a lane when D
        // allows; the row stays packed in 4 registers, so the per-row work of
        // a lane group covers twice the columns (with the edge term's
        // separate pass in the reduce: c4 backward 296 -> 282 us in the
        // fwd+bwd step)
        if (g16 && g_align16 && D % 8 == 0 && tuning(PLE_TUNE_BWD_VEC) != 4) vec = 8;
        if (tuning(PLE_TUNE_BWD_VEC) == 1) vec = 1;
        const int uv = static_cast<int>(D / vec);
        int lgw = 2;
        while (lgw < uv) lgw *= 2;
        if (lgw <= kWave) {
            const int LG = kBlock / lgw;
            int best_fs = 0;
            size_t best_lds = 0;
            BwdArgs geo{};
            auto pm_for = [&](int fs, int64_t bw) { return kP / kL + static_cast<int>(std::min<int64_t>(kP, fs * bw)); };
            int bw = static_cast<int>(std::min<int64_t>(B, 4096)), nw = 1;
            for (int fs = 4; fs >= 1 && B <= 4096; fs /= 2) {
                if ((fs > 1 && fs > F) || static_cast<int64_t>(fs) * B >= 65536) continue;
                BwdArgs t{};
                const size_t lds = reduce_layout(t, fs, static_cast<int>(B), static_cast<int>(D), LG, pm_for(fs, B), raw_db, lin);
                if (lds <= kReduceLdsTarget || (fs == 1 && lds <= kLdsMax)) {
                    best_fs = fs;
                    best_lds = lds;
                    geo = t;
                    break;
                }
            }
            const int fs_env = tuning(PLE_TUNE_BWD_FS);
            if ((fs_env == 1 || fs_env == 2 || fs_env == 4 || fs_env == 8 || fs_env == 16) && B <= 4096 &&
                static_cast<int64_t>(fs_env) * B < 65536) {
                BwdArgs t{};
                const size_t lds = reduce_layout(t, fs_env, static_cast<int>(B), static_cast<int>(D), LG, pm_for(fs_env, B), raw_db, lin);
                if (lds <= kLdsMax) {
                    best_fs = fs_env;
                    best_lds = lds;
                    geo = t;
                }
            }
            // Tables beyond LDS (or beyond 4096 bins): windows of bins, one
            // feature a workgroup, as wide as two workgroups per CU allow,
            // then evened out over the bins.  Every window ranks all pairs
            // of its sub-tiles and reduces those of its bins, so the gradient
            // is still read once; the bin indices and x once per window.
            // Windows split a feature's per-feature sums (raw-gradient bias,
            // linear0), so those plans keep the fallback kernels.
            if (best_fs == 0 && !raw_db && !lin) {
                auto lds_of = [&](BwdArgs &t, int w) {
                    return reduce_layout(t, 1, w, static_cast<int>(D), LG, pm_for(1, w), raw_db, lin);
                };
                int lo = 1, hi = static_cast<int>(std::min<int64_t>(B, 4096));
                BwdArgs t{};
                if (lds_of(t, lo) <= kReduceLdsTarget) {
                    while (lo < hi) {   // the widest window within the target
                        const int mid = (lo + hi + 1) / 2;
                        if (lds_of(t, mid) <= kReduceLdsTarget) lo = mid;
                        else hi = mid - 1;
                    }
                    nw = static_cast<int>((B + lo - 1) / lo);
                    bw = static_cast<int>((B + nw - 1) / nw);
                    best_fs = 1;
                    best_lds = lds_of(t, bw);
                    geo = t;
                }
            }
            int rb = kBlock;
            if (best_fs > 0) {
                const int PM = pm_for(best_fs, nw > 1 ? bw : B);
                // Twice the workgroup size where LDS leaves room for one
                // reduce workgroup per CU (fp32 gradient and quantisation, no
                // linear0 branch): c2 -20 us; where two fit, the wide form
                // measured slower (c3 +28 us, c4 +190 us).
                {
                    const bool wide_ok = !raw_db && !g16 && !lin;
                    bool wide = wide_ok && kLdsMax / best_lds < 2;
                    const int rb_env = tuning(PLE_TUNE_BWD_RB);
                    if (rb_env == kBlock || rb_env == kWideBlock) wide = wide_ok && rb_env == kWideBlock;
                    if (wide) {
                        BwdArgs tw = geo;
                        const size_t ldsw = reduce_layout(tw, best_fs, nw > 1 ? bw : static_cast<int>(B),
                                                          static_cast<int>(D), kWideBlock / lgw, PM, raw_db, lin);
                        if (ldsw <= kLdsMax) {
                            geo = tw;
                            best_lds = ldsw;
                            rb = kWideBlock;
                        }
                    }
                }
                {
                    pl.sorted = true;
                    pl.vec = vec;
                    pl.rb = rb;
                    pl.lds = best_lds;
                    geo.FS = best_fs;
                    geo.BW = nw > 1 ? bw : static_cast<int>(B);
                    geo.NW = nw;
                    geo.G = static_cast<int>((F + best_fs - 1) / best_fs) * nw;
                    geo.NT = kP / best_fs;
                    geo.T = static_cast<int>((N + geo.NT - 1) / geo.NT);
                    geo.PM = PM;
                    geo.LGW = lgw;
                    // chunks of sub-tiles: as many workgroups as the CUs
                    // hold at once (registers allow two 256-thread or one
                    // 512-thread workgroup per CU; LDS may allow fewer), so
                    // that every workgroup starts in the first round, within
                    // the partials budget.  More rounds (the
                    // PLE_TUNE_BWD_WG_PER_CU knob) measured slower: each
                    // workgroup stages its tables and writes its partials.
                    const int64_t per_chunk = F * B * 2 * D * 4;
                    const int resident = rb == kWideBlock ? 1 : static_cast<int>(std::min<size_t>(2, kLdsMax / best_lds));
                    const int wg_k = tuning(PLE_TUNE_BWD_WG_PER_CU);
                    int64_t c = (static_cast<int64_t>(wg_k > 0 ? wg_k : resident) * cus + geo.G - 1) / geo.G;
                    const int64_t budget_c = static_cast<int64_t>(kPartialBudget) / per_chunk;
                    if (c > budget_c) c = budget_c;
                    if (c > geo.T) c = geo.T;
                    if (c < 1) c = 1;
                    geo.SPC = static_cast<int>((geo.T + c - 1) / c);
                    pl.C = pl.Cd = (geo.T + geo.SPC - 1) / geo.SPC;
                    pl.NC = static_cast<int64_t>(geo.SPC) * geo.NT;
                    pl.geo = geo;
                }
            }
        }
    }
    if (!pl.sorted) {
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
        // histogram cells (of one block of up to 64 columns) in LDS when they
        // fit, else in the partials themselves
        pl.lds = static_cast<size_t>(B) * std::min<int64_t>(D, kWave) * 2 * sizeof(float);
        pl.hist_global = pl.lds > kLdsMax || tuning(PLE_TUNE_BWD_SIMPLE_GLOBAL) == 1;
        if (pl.hist_global) pl.lds = 0;
    }
    // A sorted plan of one chunk and one window writes dW and db from the
    // gradient kernel's LDS histogram (no chunk partials); other plans keep
    // per-chunk partials.
    if (!(pl.sorted && pl.C == 1 && pl.geo.NW == 1)) {
        pl.part_bytes = static_cast<size_t>(pl.Cd) * F * B * 2 * D * sizeof(float);
        pl.part_db_bytes = static_cast<size_t>(pl.Cd) * F * D * sizeof(float);
        pl.part_lw_bytes = lin ? static_cast<size_t>(pl.Cd) * F * D * sizeof(float) : 0;
    }
    return pl;
}

// Plans depend only on the shape, the gradient's alignment, the epilogue
// flags, the device's CU count and the tuning knobs: a small per-thread cache
// keeps the planner off the per-launch path.
const BwdPlan &plan_cached(int64_t N, int64_t F, int64_t B, int64_t D, bool g_align16, bool g16, bool raw_db,
                           bool lin) {
    struct Entry {
        int64_t N, F, B, D;
        int flags, cus;
        uint32_t epoch;
        bool valid;
        BwdPlan pl;
    };
    constexpr int kEntries = 8;
    thread_local Entry cache[kEntries] = {};
    thread_local int next = 0;
    const int cus = device_cu_count();
    const uint32_t epoch = tuning_epoch();
    const int flags = (g_align16 ? 1 : 0) | (raw_db ? 2 : 0) | (lin ? 4 : 0) | (g16 ? 8 : 0);
    for (const Entry &e : cache)
        if (e.valid && e.N == N && e.F == F && e.B == B && e.D == D && e.flags == flags && e.cus == cus &&
            e.epoch == epoch)
            return e.pl;
    Entry &e = cache[next];
    next = (next + 1) % kEntries;
    e.N = N; e.F = F; e.B = B; e.D = D; e.flags = flags; e.cus = cus; e.epoch = epoch;
    e.pl = plan_backward(N, F, B, D, g_align16, g16, raw_db, lin);
    e.valid = true;
    return e.pl;
}

// Timer events of the backward's gradient kernels being issued
// (launch_typed sets them; both NULL unless kernel timing is on).
thread_local TimerSlot t_slot;

template <typename K>
void launch_bwd(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, const BwdArgs &a) {
    hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), s, t_slot.start, t_slot.stop, 0u, a);
}

template <int GD, int NBT>
void launch_mfma(int nq, dim3 grid, size_t lds, hipStream_t s, const BwdArgs &a) {
    switch (nq) {
        case 1: launch_bwd((ple_bwd_mfma_kernel<GD, NBT, 1>), grid, dim3(kMfmaBlock), lds, s, a); break;
        case 2: launch_bwd((ple_bwd_mfma_kernel<GD, NBT, 2>), grid, dim3(kMfmaBlock), lds, s, a); break;
        case 3: launch_bwd((ple_bwd_mfma_kernel<GD, NBT, 3>), grid, dim3(kMfmaBlock), lds, s, a); break;
        default: launch_bwd((ple_bwd_mfma_kernel<GD, NBT, 4>), grid, dim3(kMfmaBlock), lds, s, a); break;
    }
}

// Lane-group width as a template argument (DPP reductions) for the 4- and
// 2-float rows and the common one-column-a-lane widths; the other widths of
// one column a lane take it at run time.
template <int GD, int Q, int EPI, int RB>
hipError_t launch_reduce_epi(const BwdArgs &a, int vec, dim3 grid, size_t lds, hipStream_t s) {
    const dim3 blk(RB);
    constexpr int esz = GD == PLE_DTYPE_F32 ? 4 : 2;
    constexpr int SH = EPI | kBwdShared;
    const bool shared = (static_cast<int64_t>(a.D) * esz) % 128 != 0;   // rows end inside a line
    if (vec == 8) {
        // (16-bit gradients only, D a multiple of 8: groups of 2 to 8 lanes;
        // rows wider than 64 columns -- no module epilogue there -- 16 to 64)
        if constexpr (GD != PLE_DTYPE_F32) {
            switch (a.LGW) {
                case 2: launch_bwd((ple_bwd_fused_kernel<GD, Q, 8, 2, EPI, RB>), grid, blk, lds, s, a); break;
                case 4: launch_bwd((ple_bwd_fused_kernel<GD, Q, 8, 4, EPI, RB>), grid, blk, lds, s, a); break;
                case 8:
                    if (shared) launch_bwd((ple_bwd_fused_kernel<GD, Q, 8, 8, SH, RB>), grid, blk, lds, s, a);
                    else launch_bwd((ple_bwd_fused_kernel<GD, Q, 8, 8, EPI, RB>), grid, blk, lds, s, a);
                    break;
                default:
                    if constexpr (EPI == 0) {
                        if (a.LGW == 16) launch_bwd((ple_bwd_fused_kernel<GD, Q, 8, 16, 0, RB>), grid, blk, lds, s, a);
                        else if (a.LGW == 32) launch_bwd((ple_bwd_fused_kernel<GD, Q, 8, 32, 0, RB>), grid, blk, lds, s, a);
                        else launch_bwd((ple_bwd_fused_kernel<GD, Q, 8, 64, 0, RB>), grid, blk, lds, s, a);
                        break;
                    } else {
                        return hipErrorInvalidConfiguration;
                    }
            }
            return hipGetLastError();
        } else {
            return hipErrorInvalidConfiguration;
        }
    }
    if (vec == 4) {
        // rows of more than 64 columns (no module epilogue there): 32- and
        // 64-lane groups
        if (a.LGW > 16) {
            if constexpr (EPI == 0) {
                if (a.LGW == 32) launch_bwd((ple_bwd_fused_kernel<GD, Q, 4, 32, 0, RB>), grid, blk, lds, s, a);
                else launch_bwd((ple_bwd_fused_kernel<GD, Q, 4, 64, 0, RB>), grid, blk, lds, s, a);
                return hipGetLastError();
            } else {
                return hipErrorInvalidConfiguration;
            }
        }
        switch (a.LGW) {
            case 2: launch_bwd((ple_bwd_fused_kernel<GD, Q, 4, 2, EPI, RB>), grid, blk, lds, s, a); break;
            case 4: launch_bwd((ple_bwd_fused_kernel<GD, Q, 4, 4, EPI, RB>), grid, blk, lds, s, a); break;
            case 8:
                // (16-bit rows of 8-lane groups are not streamed: no twin)
                if constexpr (GD == PLE_DTYPE_F32) {
                    if (shared) {
                        launch_bwd((ple_bwd_fused_kernel<GD, Q, 4, 8, SH, RB>), grid, blk, lds, s, a);
                        break;
                    }
                }
                launch_bwd((ple_bwd_fused_kernel<GD, Q, 4, 8, EPI, RB>), grid, blk, lds, s, a);
                break;
            default:
                if (shared) launch_bwd((ple_bwd_fused_kernel<GD, Q, 4, 16, SH, RB>), grid, blk, lds, s, a);
                else launch_bwd((ple_bwd_fused_kernel<GD, Q, 4, 16, EPI, RB>), grid, blk, lds, s, a);
                break;
        }
    } else if (vec == 2) {
        // (the planner takes 2 per lane for 6 <= D <= 64: groups of 4 to 32 lanes)
        switch (a.LGW) {
            case 4: launch_bwd((ple_bwd_fused_kernel<GD, Q, 2, 4, EPI, RB>), grid, blk, lds, s, a); break;
            case 8: launch_bwd((ple_bwd_fused_kernel<GD, Q, 2, 8, EPI, RB>), grid, blk, lds, s, a); break;
            case 16: launch_bwd((ple_bwd_fused_kernel<GD, Q, 2, 16, EPI, RB>), grid, blk, lds, s, a); break;
            case 32: launch_bwd((ple_bwd_fused_kernel<GD, Q, 2, 32, EPI, RB>), grid, blk, lds, s, a); break;
            default: return hipErrorInvalidConfiguration;
        }
    } else {
        // one column a lane: DPP group sums for the 16- to 64-lane groups
        // (9 <= D <= 64), shuffles at run time for the others
        switch (a.LGW) {
            case 16: launch_bwd((ple_bwd_fused_kernel<GD, Q, 1, 16, EPI, RB>), grid, blk, lds, s, a); break;
            case 32: launch_bwd((ple_bwd_fused_kernel<GD, Q, 1, 32, EPI, RB>), grid, blk, lds, s, a); break;
            case 64: launch_bwd((ple_bwd_fused_kernel<GD, Q, 1, 64, EPI, RB>), grid, blk, lds, s, a); break;
            default: launch_bwd((ple_bwd_fused_kernel<GD, Q, 1, 0, EPI, RB>), grid, blk, lds, s, a); break;
        }
    }
    return hipGetLastError();
}

// rb: the reduce workgroup size, kBlock or kWideBlock (fp32 gradient and
// quantisation, no linear0 branch; the planner picks it).
template <int GD, int Q>
hipError_t launch_reduce(const BwdArgs &a, int vec, int epi, int rb, dim3 grid, size_t lds, hipStream_t s) {
    if (rb == kWideBlock) {
        if constexpr (GD == PLE_DTYPE_F32 && Q == PLE_DTYPE_F32) {
            if (epi == 0) return launch_reduce_epi<GD, Q, 0, kWideBlock>(a, vec, grid, lds, s);
            if (epi == kBwdRelu) return launch_reduce_epi<GD, Q, kBwdRelu, kWideBlock>(a, vec, grid, lds, s);
        }
        return hipErrorInvalidConfiguration;   // (the planner never asks for it elsewhere)
    }
    if constexpr (GD == PLE_DTYPE_F32) {
        // module epilogues (their gradient is fp32)
        switch (epi) {
            case kBwdRelu: return launch_reduce_epi<GD, Q, kBwdRelu, kBlock>(a, vec, grid, lds, s);
            case kBwdLin: return launch_reduce_epi<GD, Q, kBwdLin, kBlock>(a, vec, grid, lds, s);
            case kBwdLin | kBwdRelu:
                return launch_reduce_epi<GD, Q, kBwdLin | kBwdRelu, kBlock>(a, vec, grid, lds, s);
            default: break;
        }
    }
    return launch_reduce_epi<GD, Q, 0, kBlock>(a, vec, grid, lds, s);
}

template <int GD, int Q>
hipError_t launch_typed(BwdArgs a, const BwdPlan &pl, int idxb, bool want_dx, bool want_dwdb, hipStream_t s) {
    hipError_t e = hipSuccess;
    const int epi = (a.mask ? kBwdRelu : 0) | (a.lin_w ? kBwdLin : 0);
    if (pl.mfma_nbt > 0) {
        // (planned only for a 16-bit gradient in its own dtype, no epilogue,
        // uint8 bin indices)
        if constexpr (GD != PLE_DTYPE_F32 && GD == Q) {
            if (epi != 0 || idxb != 1) return hipErrorInvalidConfiguration;
            a.db_from_buckets = 1;
            a.fin_fused = want_dwdb && pl.C == 1;
            const dim3 grid(static_cast<unsigned>(kNumXcd * tiles_per_xcd(a.G, pl.C)));
            const TimerSlot ts = timer_slot(PLE_TIMER_BACKWARD);
            t_slot = ts;
            switch (pl.mfma_nbt) {
                case 1: launch_mfma<GD, 1>(pl.mfma_nq, grid, pl.lds, s, a); break;
                case 2: launch_mfma<GD, 2>(pl.mfma_nq, grid, pl.lds, s, a); break;
                default: launch_mfma<GD, 3>(pl.mfma_nq, grid, pl.lds, s, a); break;
            }
            t_slot = TimerSlot{};
            e = hipGetLastError();
            if (e != hipSuccess) return e;
            timer_commit(ts);
        } else {
            return hipErrorInvalidConfiguration;
        }
    } else if (pl.sorted) {
        // (linear0's bias gradient without a ReLU: the buckets sum the unmasked g)
        a.db_from_buckets = (Q == PLE_DTYPE_F32 || GD == Q) && (a.lin_w == nullptr || a.mask == nullptr);
        const dim3 grid(static_cast<unsigned>(kNumXcd * tiles_per_xcd(a.G, pl.C)));
        a.idxb = idxb;
        // one chunk (and one window): the gradient kernel writes dW / db itself
        a.fin_fused = want_dwdb && pl.C == 1 && a.NW == 1;
        const TimerSlot ts = timer_slot(PLE_TIMER_BACKWARD);
        t_slot = ts;
        e = launch_reduce<GD, Q>(a, pl.vec, epi, pl.rb, grid, pl.lds, s);
        t_slot = TimerSlot{};
        if (e != hipSuccess) return e;
        timer_commit(ts);
    } else {
        // timed from the start of the first kernel to the end of the last
        const TimerSlot ts = timer_slot(PLE_TIMER_BACKWARD);
        if (want_dx) {
            t_slot = TimerSlot{ts.start, want_dwdb ? nullptr : ts.stop};
            const int64_t pairs = a.N * a.F;
            int64_t blocks = (pairs + (kBlock / 16) - 1) / (kBlock / 16);
            const int64_t cap = static_cast<int64_t>(device_cu_count()) * 16;
            if (blocks > cap) blocks = cap;
            if (blocks < 1) blocks = 1;
            if (idxb == 1) launch_bwd((ple_bwd_simple_dx_kernel<GD, Q, uint8_t>), dim3(blocks), dim3(kBlock), 0, s, a);
            else if (idxb == 2) launch_bwd((ple_bwd_simple_dx_kernel<GD, Q, int16_t>), dim3(blocks), dim3(kBlock), 0, s, a);
            else launch_bwd((ple_bwd_simple_dx_kernel<GD, Q, int32_t>), dim3(blocks), dim3(kBlock), 0, s, a);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        if (want_dwdb) {
            t_slot = TimerSlot{want_dx ? nullptr : ts.start, ts.stop};
            const int64_t col_blocks = (a.D + kWave - 1) / kWave;
            const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.F) * pl.C * col_blocks));
            if (pl.hist_global) {
                if (idxb == 1) launch_bwd((ple_bwd_simple_hist_kernel<GD, Q, uint8_t, true>), grid, dim3(kWave), 0, s, a);
                else if (idxb == 2) launch_bwd((ple_bwd_simple_hist_kernel<GD, Q, int16_t, true>), grid, dim3(kWave), 0, s, a);
                else launch_bwd((ple_bwd_simple_hist_kernel<GD, Q, int32_t, true>), grid, dim3(kWave), 0, s, a);
            } else {
                if (idxb == 1) launch_bwd((ple_bwd_simple_hist_kernel<GD, Q, uint8_t, false>), grid, dim3(kWave), pl.lds, s, a);
                else launch_bwd((ple_bwd_simple_hist_kernel<GD, Q, int16_t, false>), grid, dim3(kWave), pl.lds, s, a);
            }
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        t_slot = TimerSlot{};
        timer_commit(ts);
    }
    if (want_dwdb && !((pl.sorted || pl.mfma_nbt > 0) && a.fin_fused)) {
        size_t lds = static_cast<size_t>(a.B) * 2 * kFinStride * sizeof(float);
        a.fin_direct = lds > kLdsMax;          // very many bins: no LDS table
        if (a.fin_direct) lds = 0;
        // The finalize sums the chunks itself unless a thread would issue more
        // than kFinLoadsInline loads; then a wide kernel sums them first.
        const int64_t loads = static_cast<int64_t>(a.B) * 2 * kFinCols * a.Cd / kBlock;
        a.fin_summed = a.Cd > 1 && (a.fin_direct || loads > kFinLoadsInline);
        if (a.fin_summed) {
            const int64_t per_chunk = static_cast<int64_t>(a.F) * a.B * 2 * a.D;
            int64_t blocks = (per_chunk + kBlock - 1) / kBlock;
            const int64_t cap = static_cast<int64_t>(device_cu_count()) * 32;
            if (blocks > cap) blocks = cap;
            hipLaunchKernelGGL(ple_bwd_chunksum_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, a.part,
                               per_chunk, a.Cd);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        const dim3 fg(static_cast<unsigned>(a.F), static_cast<unsigned>((a.D + kFinCols - 1) / kFinCols));
        hipLaunchKernelGGL(ple_bwd_finalize_kernel, fg, dim3(kBlock), lds, s, a);
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
    // the plan depends on the gradient's alignment and dtype; report the largest need
    // (and on the epilogue: the linear0 sums need their own partials).  The
    // last few answers are kept per thread.
    struct Entry {
        int64_t N, F, B, D;
        int cus;
        uint32_t epoch;
        size_t bytes;
    };
    constexpr int kEntries = 4;
    thread_local Entry cache[kEntries] = {};
    thread_local int next = 0;
    const int cus = device_cu_count();
    const uint32_t epoch = tuning_epoch();
    for (const Entry &e : cache)
        if (e.cus == cus && e.N == N && e.F == F && e.B == B && e.D == D && e.epoch == epoch) return e.bytes;
    size_t need = 0;
    for (int al = 0; al < 2; ++al)
        for (int g16 = 0; g16 < 2; ++g16)
            for (int raw = 0; raw < 2; ++raw)
                for (int lin = 0; lin < 2; ++lin) {
                    const size_t t = plan_backward(N, F, B, D, al != 0, g16 != 0, raw != 0, lin != 0).total();
                    need = t > need ? t : need;
                }
    cache[next] = Entry{N, F, B, D, cus, epoch, need};
    next = (next + 1) % kEntries;
    return need;
}

int backward_plan_info(const BackwardRequest &r, ple_backward_plan_info_t *info) {
    const bool lin = r.lin_w != nullptr;
    const bool raw_db = (r.quant != PLE_DTYPE_F32 && r.quant != r.grad_dtype) || (lin && r.relu);
    const uintptr_t gaddr = reinterpret_cast<uintptr_t>(r.g);
    const BwdPlan &pl = plan_cached(r.N, r.F, r.B, r.D, gaddr % 16 == 0, r.grad_dtype != PLE_DTYPE_F32, raw_db, lin);
    info->sorted = pl.sorted ? 1 : 0;
    info->chunks = pl.C;
    info->features_per_group = pl.sorted || pl.mfma_nbt > 0 ? pl.geo.FS : 1;
    info->columns_per_lane = pl.sorted ? pl.vec : 1;
    info->lanes_per_row = pl.sorted ? pl.geo.LGW : 1;
    info->threads = pl.sorted || pl.mfma_nbt > 0 ? pl.rb : kWave;
    info->lds_bytes = pl.lds;
    info->workspace_bytes = pl.total();
    info->bins_per_window = pl.sorted ? pl.geo.BW : static_cast<int>(r.B);
    info->windows = pl.sorted ? pl.geo.NW : 1;
    info->matrix_cores = pl.mfma_nbt > 0 ? 1 : 0;
    return PLE_OK;
}

int backward_run(const BackwardRequest &r) {
    const bool lin = r.lin_w != nullptr;
    const bool want_dx = r.dx != nullptr;
    const bool want_dwdb = r.dw != nullptr || r.db != nullptr || r.dlw != nullptr;
    if (r.grad_dtype != PLE_DTYPE_F32 && r.quant != r.grad_dtype) return PLE_E_UNSUPPORTED;
    // module epilogues: fp32 gradient; a ReLU needs the forward's bits
    if ((r.relu || lin) && r.grad_dtype != PLE_DTYPE_F32) return PLE_E_UNSUPPORTED;
    if (r.relu && !r.mask) return PLE_E_NULL_POINTER;
    // module epilogues: rows of at most 64 columns (the module's limit on
    // d_embedding; the forward gathers the ReLU pass bits of a row's lanes)
    if ((r.relu || lin) && r.D > 64) return PLE_E_TOO_LARGE;
    if (r.dlw && !lin) return PLE_E_UNSUPPORTED;
    const uintptr_t gaddr = reinterpret_cast<uintptr_t>(r.g);
    const int gbytes = r.grad_dtype == PLE_DTYPE_F32 ? 4 : 2;
    if (gaddr % gbytes != 0) return PLE_E_MISALIGNED;
    // (a gradient in the quantisation dtype is its own rounding: its bias
    // gradient is the sum of the buckets, as for fp32)
    const bool raw_db = (r.quant != PLE_DTYPE_F32 && r.quant != r.grad_dtype) || (lin && r.relu);
    const BwdPlan &pl = plan_cached(r.N, r.F, r.B, r.D, gaddr % 16 == 0, r.grad_dtype != PLE_DTYPE_F32, raw_db, lin);
    // The workspace holds chunk partials of dW / db only (the sorted path's
    // descriptors live in LDS): dx alone needs none.
    const size_t need = want_dwdb ? pl.total() : 0;
    if (need > 0 && (r.workspace == nullptr || r.workspace_bytes < need ||
                     reinterpret_cast<uintptr_t>(r.workspace) % 256 != 0))
        return PLE_E_WORKSPACE;
    const int64_t grid_max = pl.sorted || pl.mfma_nbt > 0 ? kNumXcd * tiles_per_xcd(pl.geo.G, pl.C)
                                       : static_cast<int64_t>(r.F) * pl.C * ((r.D + kWave - 1) / kWave);
    if (grid_max > INT32_MAX) return PLE_E_TOO_LARGE;
    BwdArgs a = pl.geo;
    a.g = r.g; a.x = r.x; a.edges = r.edges; a.iw = r.iw; a.nbins = r.nbins; a.weight = r.weight;
    a.idx = r.idx; a.dx = r.dx; a.dw = r.dw; a.db = r.db;
    a.mask = r.relu ? r.mask : nullptr; a.MW = static_cast<int>((r.D + 31) / 32);
    a.lin_w = r.lin_w; a.dlw = r.dlw;
    char *ws = static_cast<char *>(r.workspace);
    size_t off = 0;
    auto carve = [&](size_t bytes) {
        char *p = ws + off;
        off += align_up(bytes, 256);
        return p;
    };
    float *part = reinterpret_cast<float *>(carve(pl.part_bytes));
    float *part_db = reinterpret_cast<float *>(carve(pl.part_db_bytes));
    float *part_lw = reinterpret_cast<float *>(carve(pl.part_lw_bytes));
    a.part = want_dwdb ? part : nullptr;
    a.part_db = want_dwdb ? part_db : nullptr;
    a.part_lw = want_dwdb && lin ? part_lw : nullptr;
    if (!want_dx) a.dx = nullptr;
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
