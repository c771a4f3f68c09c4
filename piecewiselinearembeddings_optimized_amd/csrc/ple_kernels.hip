// MI355X (gfx950) kernels for the fused piecewise-linear-embedding path and
// the C ABI declared in include/ple_hip.h.
//
// Written for CDNA4: 64-lane wavefronts, 160 KiB of LDS per CU, 256 CUs in 8
// XCDs with one L2 each.  The path is HBM-bound (about one fma per stored
// element), so the kernels are organised around streaming the [N, F, D]
// tensor once with wide coalesced accesses; no MFMA.
//
// Forward (ple_fwd_kernel): one workgroup owns a group of FS features and a
// chunk of samples.  It stages, per feature, the bin edges, the inverse
// widths and a [bins x 2D] table {prefix of quantised weights | quantised
// weight row} in LDS, then streams wave tiles of 64 (sample, feature) pairs:
// each lane bin-searches one pair in LDS, the pair's (bin, fraction) is handed
// to the lanes that store that pair's D outputs through ds_bpermute, and the
// outputs go out as 16-byte stores covering whole sample rows of the group.
//
// Backward: a dx kernel (one lane group per pair), a per-(feature, sample
// chunk) histogram kernel that accumulates the bucket / weighted sums of the
// gradient per bin in LDS in sample order (each LDS cell has exactly one
// owning lane), and a finalize kernel that sums the chunk partials in chunk
// order and takes the suffix over bins.  Every floating-point reduction has a
// fixed order, so results are bitwise reproducible.

#include <hip/hip_runtime.h>

#include <stddef.h>
#include <stdint.h>

#include "../../include/ple_hip.h"

namespace {

constexpr int kWave = 64;
constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kNumXcd = 8;

// ---------------------------------------------------------------------------
// element helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_round(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return __uint_as_float(0x7fc00000u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return __uint_as_float(u & 0xffff0000u);
}

// Only called on values already rounded by bf16_round (low half is zero).
__device__ __forceinline__ uint16_t bf16_bits_of_rounded(float v) {
    return static_cast<uint16_t>(__float_as_uint(v) >> 16);
}

__device__ __forceinline__ float f16_round(float v) {
    return static_cast<float>(static_cast<_Float16>(v));
}

__device__ __forceinline__ uint16_t f16_bits(float v) {
    _Float16 h = static_cast<_Float16>(v);
    return __builtin_bit_cast(uint16_t, h);
}

template <int Q>
__device__ __forceinline__ float quant(float v) {
    if constexpr (Q == PLE_DTYPE_BF16) return bf16_round(v);
    else if constexpr (Q == PLE_DTYPE_F16) return f16_round(v);
    else return v;
}

template <int G>
__device__ __forceinline__ float load_grad(const void *p, int64_t i) {
    if constexpr (G == PLE_DTYPE_F32) {
        return static_cast<const float *>(p)[i];
    } else if constexpr (G == PLE_DTYPE_BF16) {
        uint32_t b = static_cast<const uint16_t *>(p)[i];
        return __uint_as_float(b << 16);
    } else {
        uint16_t b = static_cast<const uint16_t *>(p)[i];
        return static_cast<float>(__builtin_bit_cast(_Float16, b));
    }
}

// searchsorted(edges[0..n], v, side=right) - 1, clamped to [0, n-1].  Every
// comparison with NaN is false, so NaN walks to the top and lands in bin n-1.
__device__ __forceinline__ int find_bin(float v, const float *e, int n) {
    int lo = 0;
    int hi = n + 1;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (v < e[mid]) hi = mid;
        else lo = mid + 1;
    }
    int k = lo - 1;
    k = k < 0 ? 0 : k;
    k = k > n - 1 ? n - 1 : k;
    return k;
}

// n_bins and bin indices come from the caller; clamping them keeps every
// table access inside its row even for inconsistent inputs (valid inputs are
// unchanged).
__device__ __forceinline__ int clamp_nbins(int n, int bmax) {
    return n < 1 ? 1 : (n > bmax ? bmax : n);
}

__device__ __forceinline__ int clamp_bin(int k, int n) {
    return k < 0 ? 0 : (k > n - 1 ? n - 1 : k);
}

__device__ __forceinline__ int phys_bin(int k, int n, int bmax) {
    return k == n - 1 ? bmax - 1 : k;
}

template <typename IdxT>
__device__ __forceinline__ int load_idx(const void *p, int64_t i) {
    return static_cast<int>(static_cast<const IdxT *>(p)[i]);
}

// Stores VEC consecutive outputs (VEC in {1, 4}).
template <int OUT, int VEC>
__device__ __forceinline__ void store_out(void *base, int64_t i, const float *v) {
    if constexpr (OUT == PLE_DTYPE_F32) {
        float *p = static_cast<float *>(base) + i;
        if constexpr (VEC == 4) {
            *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
            p[0] = v[0];
        }
    } else {
        uint16_t h[VEC];
#pragma unroll
        for (int t = 0; t < VEC; ++t) {
            if constexpr (OUT == PLE_DTYPE_BF16) h[t] = bf16_bits_of_rounded(bf16_round(v[t]));
            else h[t] = f16_bits(v[t]);
        }
        uint16_t *p = static_cast<uint16_t *>(base) + i;
        if constexpr (VEC == 4) {
            uint2 w;
            w.x = static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
            w.y = static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16);
            *reinterpret_cast<uint2 *>(p) = w;
        } else {
            p[0] = h[0];
        }
    }
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------

struct FwdArgs {
    const float *x;
    const float *edges;
    const float *iw;
    const int32_t *nbins;
    const float *weight;
    const float *bias;
    void *out;
    void *idx;
    int64_t N;
    int F, B, D;
    int FS;       // features per workgroup (power of two, FS * D/VEC <= 64)
    int G;        // feature groups = ceil(F / FS)
    int C;        // sample chunks (multiple of kNumXcd)
    int64_t NC;   // samples per chunk
};

__host__ __device__ inline size_t fwd_lds_floats(int FS, int B, int D) {
    return static_cast<size_t>(FS) * B * 2 * D      // table {prefix | weight}
         + static_cast<size_t>(FS) * (B + 1)        // edges
         + static_cast<size_t>(FS) * B              // inverse widths
         + static_cast<size_t>(FS);                 // n_bins
}

// Workgroup -> (feature group, sample chunk), XCD aware: workgroup ids are
// dealt to the XCDs round-robin, so the chunks are dealt the same way and all
// feature groups of one chunk run back to back on one XCD.  They then share
// that XCD's L2 lines of x and of the bin indices.
__device__ __forceinline__ bool decode_tile(int bid, int G, int C, int &g, int &c) {
    const int x8 = bid % kNumXcd;
    const int L = bid / kNumXcd;
    g = L % G;
    c = (L / G) * kNumXcd + x8;
    return c < C;
}

template <int Q, int OUT, bool HAS_BIAS, int VEC, typename IdxT>
__global__ __launch_bounds__(kBlock) void ple_fwd_kernel(FwdArgs a) {
    extern __shared__ float smem[];
    const int FS = a.FS, B = a.B, D = a.D, F = a.F;
    const int rs = 2 * D;                                   // table row stride
    float *tbl = smem;
    float *sedge = tbl + static_cast<size_t>(FS) * B * rs;
    float *siw = sedge + FS * (B + 1);
    int *snb = reinterpret_cast<int *>(siw + FS * B);

    int g, c;
    if (!decode_tile(blockIdx.x, a.G, a.C, g, c)) return;
    const int f0 = g * FS;
    const int nfh = min(FS, F - f0);
    const int64_t n_begin = static_cast<int64_t>(c) * a.NC;
    const int64_t n_end = min(a.N, n_begin + a.NC);
    if (n_begin >= n_end) return;
    const int tid = threadIdx.x;

    // ---- stage the per-feature tables ------------------------------------
    for (int i = tid; i < FS; i += kBlock) snb[i] = i < nfh ? clamp_nbins(a.nbins[f0 + i], B) : 1;
    for (int i = tid; i < FS * (B + 1); i += kBlock) {
        const int fl = i / (B + 1);
        sedge[i] = fl < nfh ? a.edges[static_cast<int64_t>(f0) * (B + 1) + i] : 0.0f;
    }
    for (int i = tid; i < FS * B; i += kBlock) {
        const int fl = i / B;
        siw[i] = fl < nfh ? a.iw[static_cast<int64_t>(f0) * B + i] : 0.0f;
    }
    __syncthreads();

    const int U = D / VEC;
    for (int i = tid; i < FS * B * U; i += kBlock) {
        const int fl = i / (B * U);
        const int r = i - fl * (B * U);
        const int k = r / U;
        const int u = r - k * U;
        if (fl < nfh) {
            const int n = snb[fl];
            if (k < n) {
                const int p = phys_bin(k, n, B);
                const float *src = a.weight + ((static_cast<int64_t>(f0 + fl) * B + p) * D + u * VEC);
                float *dst = tbl + (static_cast<size_t>(fl) * B + k) * rs + D + u * VEC;
                if constexpr (VEC == 4) {
                    float4 w = *reinterpret_cast<const float4 *>(src);
                    dst[0] = quant<Q>(w.x);
                    dst[1] = quant<Q>(w.y);
                    dst[2] = quant<Q>(w.z);
                    dst[3] = quant<Q>(w.w);
                } else {
                    dst[0] = quant<Q>(src[0]);
                }
            }
        }
    }
    __syncthreads();

    // prefix over logical bins, one lane per (feature, column), in bin order
    for (int col = tid; col < FS * D; col += kBlock) {
        const int fl = col / D;
        const int j = col - fl * D;
        if (fl < nfh) {
            const int n = snb[fl];
            float *base = tbl + static_cast<size_t>(fl) * B * rs;
            float acc = 0.0f;
            int k = 0;
            for (; k + 8 <= n; k += 8) {
                float w[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) w[t] = base[(k + t) * rs + D + j];
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    base[(k + t) * rs + j] = acc;
                    acc += w[t];
                }
            }
            for (; k < n; ++k) {
                const float w = base[k * rs + D + j];
                base[k * rs + j] = acc;
                acc += w;
            }
        }
    }
    __syncthreads();

    // ---- stream wave tiles -------------------------------------------------
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int SW = kWave / FS;      // samples per wave tile
    const int Lv = FS * U;          // vector slots per sample row of the group
    const int R = kWave / Lv;       // sample rows per store instruction

    // pair phase: lane -> (sample p_s, feature p_fl)
    const int p_s = lane / FS;
    const int p_fl = lane - p_s * FS;
    const float *e_row = sedge + p_fl * (B + 1);
    const float *iw_row = siw + p_fl * B;
    const int p_n = snb[p_fl];
    const bool p_fok = p_fl < nfh;

    // store phase: lane -> (row o_s, feature o_fl, vector o_u), fixed per lane
    const int o_s = lane / Lv;
    const int o_v = lane - o_s * Lv;
    const int o_fl = o_v / U;
    const int o_u = o_v - o_fl * U;
    const bool o_ok = (o_s < R) && (o_fl < nfh);
    float bvec[VEC];
#pragma unroll
    for (int t = 0; t < VEC; ++t) bvec[t] = 0.0f;
    if constexpr (HAS_BIAS) {
        if (o_ok) {
#pragma unroll
            for (int t = 0; t < VEC; ++t)
                bvec[t] = a.bias[static_cast<int64_t>(f0 + o_fl) * D + o_u * VEC + t];
        }
    }
    const float *o_tbl = tbl + static_cast<size_t>(o_fl) * B * rs + o_u * VEC;

    const int64_t rows = n_end - n_begin;
    const int64_t n_tiles = (rows + SW - 1) / SW;
    const int64_t row_elems = static_cast<int64_t>(F) * D;

    for (int64_t t = wave; t < n_tiles; t += kWavesPerBlock) {
        const int64_t n0 = n_begin + t * SW;
        const int64_t pn = n0 + p_s;
        const bool pvalid = p_fok && (pn < n_end);
        const int64_t pidx = pn * F + f0 + p_fl;
        const float v = pvalid ? a.x[pidx] : 0.0f;
        const int k = find_bin(v, e_row, p_n);
        const float frac = (v - e_row[k]) * iw_row[k];
        const float qf = quant<Q>(frac);
        if (pvalid) static_cast<IdxT *>(a.idx)[pidx] = static_cast<IdxT>(k);

        for (int sb = 0; sb < SW; sb += R) {
            const int s = sb + o_s;
            const int src = (s * FS + o_fl) & (kWave - 1);
            const int ks = __shfl(k, src);
            const float qs = __shfl(qf, src);
            const int64_t n = n0 + s;
            if (o_ok && s < SW && n < n_end) {
                const float *row = o_tbl + static_cast<size_t>(ks) * rs;
                float r[VEC];
                if constexpr (VEC == 4) {
                    const float4 P = *reinterpret_cast<const float4 *>(row);
                    const float4 W = *reinterpret_cast<const float4 *>(row + D);
                    r[0] = fmaf(qs, W.x, P.x);
                    r[1] = fmaf(qs, W.y, P.y);
                    r[2] = fmaf(qs, W.z, P.z);
                    r[3] = fmaf(qs, W.w, P.w);
                } else {
                    r[0] = fmaf(qs, row[D], row[0]);
                }
#pragma unroll
                for (int t2 = 0; t2 < VEC; ++t2) {
                    float o = quant<Q>(r[t2]);
                    if constexpr (HAS_BIAS) o = o + bvec[t2];
                    r[t2] = o;
                }
                store_out<OUT, VEC>(a.out, n * row_elems + static_cast<int64_t>(f0 + o_fl) * D + o_u * VEC, r);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// backward: dx
// ---------------------------------------------------------------------------

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
    float *part;   // [C][F][B][2D] chunk partials {bucket | weighted}
    float *part_db;  // [C][F][D] chunk partials of the bias gradient
    float *tot;      // [F][B][2D] chunk sums {bucket | weighted}
    int64_t N;
    int F, B, D;
    int C;
    int64_t NC;
};

// One 16-lane group per (sample, feature) pair: every lane takes a strided
// slice of the D columns, then the group reduces with shuffles.
template <int GD, int Q, typename IdxT>
__global__ __launch_bounds__(kBlock) void ple_bwd_dx_kernel(BwdArgs a) {
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
        const int pk = phys_bin(k, n, B);
        const float *w = a.weight + (static_cast<int64_t>(f) * B + pk) * D;
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

// ---------------------------------------------------------------------------
// backward: per-chunk histograms
// ---------------------------------------------------------------------------

// One wave per (feature, sample chunk); lane j owns column j (D <= 64).  The
// wave walks the chunk in sample order, keeps a running sum while the bin
// repeats and folds it into its own LDS cells when the bin changes, so each
// cell is written by one lane in sample order.
template <int GD, int Q, typename IdxT>
__global__ __launch_bounds__(kWave) void ple_bwd_hist_kernel(BwdArgs a) {
    extern __shared__ float smem[];
    const int B = a.B, D = a.D, F = a.F;
    float *hb = smem;                 // [B][D] bucket
    float *hw = smem + B * D;         // [B][D] weighted
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

// One lane per (feature, bin, column): sums the chunk partials of that cell in
// chunk order into tot[F][B][2D].
__global__ __launch_bounds__(kBlock) void ple_bwd_reduce_chunks_kernel(BwdArgs a) {
    const int64_t cell = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int F = a.F, B = a.B, D = a.D;
    const int64_t per_f = static_cast<int64_t>(B) * 2 * D;
    if (cell >= static_cast<int64_t>(F) * per_f) return;
    const int f = static_cast<int>(cell / per_f);
    const int k = static_cast<int>((cell - f * per_f) / (2 * D));
    if (k >= clamp_nbins(a.nbins[f], B)) return;
    const int64_t chunk_stride = static_cast<int64_t>(F) * per_f;
    float s = 0.0f;
    for (int c = 0; c < a.C; ++c) s += a.part[c * chunk_stride + cell];
    a.tot[cell] = s;
}

// One lane per (feature, column): suffix over logical bins
// (dW[phys(k)] = weighted[k] + sum_{m>k} bucket[m]); slots no bin maps to get
// 0.  The bias gradient sums the chunk partials in chunk order.
__global__ __launch_bounds__(kBlock) void ple_bwd_finalize_kernel(BwdArgs a) {
    const int64_t col = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int F = a.F, B = a.B, D = a.D;
    if (col >= static_cast<int64_t>(F) * D) return;
    const int f = static_cast<int>(col / D);
    const int j = static_cast<int>(col - static_cast<int64_t>(f) * D);
    const int n = clamp_nbins(a.nbins[f], B);
    if (a.dw) {
        float fut = 0.0f;
        for (int k = n - 1; k >= 0; --k) {
            const float *src = a.tot + (static_cast<int64_t>(f) * B + k) * 2 * D;
            a.dw[(static_cast<int64_t>(f) * B + phys_bin(k, n, B)) * D + j] = src[D + j] + fut;
            fut += src[j];
        }
        for (int k = n - 1; k < B - 1; ++k)
            a.dw[(static_cast<int64_t>(f) * B + k) * D + j] = 0.0f;
    }
    if (a.db) {
        float s = 0.0f;
        for (int c = 0; c < a.C; ++c) s += a.part_db[(static_cast<int64_t>(c) * F + f) * D + j];
        a.db[static_cast<int64_t>(f) * D + j] = s;
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

constexpr size_t kLdsBudgetTwoPerCu = 80 * 1024;
constexpr size_t kLdsMax = 160 * 1024;

int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

int idx_bytes_for(int64_t B) { return B <= 256 ? 1 : (B <= 32768 ? 2 : 4); }

bool valid_dtype(int d) { return d == PLE_DTYPE_F32 || d == PLE_DTYPE_F16 || d == PLE_DTYPE_BF16; }

struct FwdPlan {
    int vec, FS, G, C;
    int64_t NC;
    size_t lds;
};

bool plan_forward(int64_t N, int64_t F, int64_t B, int64_t D, bool aligned16, FwdPlan &pl) {
    pl.vec = (D % 4 == 0 && aligned16) ? 4 : 1;
    const int U = static_cast<int>(D / pl.vec);
    if (U > kWave) return false;
    int fs = 1;
    while (fs * 2 <= kWave && fs * 2 * U <= kWave && fs < F) fs *= 2;
    while (fs > 1 && fwd_lds_floats(fs, static_cast<int>(B), static_cast<int>(D)) * 4 > kLdsBudgetTwoPerCu) fs /= 2;
    pl.lds = fwd_lds_floats(fs, static_cast<int>(B), static_cast<int>(D)) * 4;
    if (pl.lds > kLdsMax) return false;
    pl.FS = fs;
    pl.G = static_cast<int>((F + fs - 1) / fs);
    const int target = 8 * device_cu_count();
    int64_t c = (target + pl.G - 1) / pl.G;
    const int64_t sw = kWave / fs;
    const int64_t max_c = (N + sw - 1) / sw;          // at least one wave tile per chunk
    if (c > max_c) c = max_c;
    if (c < 1) c = 1;
    c = ((c + kNumXcd - 1) / kNumXcd) * kNumXcd;
    pl.NC = (N + c - 1) / c;
    pl.C = static_cast<int>((N + pl.NC - 1) / pl.NC);
    pl.C = ((pl.C + kNumXcd - 1) / kNumXcd) * kNumXcd;
    return true;
}

template <int Q, int OUT, bool HB, int VEC>
hipError_t launch_fwd_idx(const FwdArgs &a, int idxb, dim3 grid, size_t lds, hipStream_t s) {
    switch (idxb) {
        case 1: hipLaunchKernelGGL((ple_fwd_kernel<Q, OUT, HB, VEC, uint8_t>), grid, dim3(kBlock), lds, s, a); break;
        case 2: hipLaunchKernelGGL((ple_fwd_kernel<Q, OUT, HB, VEC, int16_t>), grid, dim3(kBlock), lds, s, a); break;
        default: hipLaunchKernelGGL((ple_fwd_kernel<Q, OUT, HB, VEC, int32_t>), grid, dim3(kBlock), lds, s, a); break;
    }
    return hipGetLastError();
}

template <int Q, int OUT, bool HB>
hipError_t launch_fwd_vec(const FwdArgs &a, int vec, int idxb, dim3 grid, size_t lds, hipStream_t s) {
    return vec == 4 ? launch_fwd_idx<Q, OUT, HB, 4>(a, idxb, grid, lds, s)
                    : launch_fwd_idx<Q, OUT, HB, 1>(a, idxb, grid, lds, s);
}

template <int Q, int OUT>
hipError_t launch_fwd_bias(const FwdArgs &a, int vec, int idxb, dim3 grid, size_t lds, hipStream_t s) {
    return a.bias ? launch_fwd_vec<Q, OUT, true>(a, vec, idxb, grid, lds, s)
                  : launch_fwd_vec<Q, OUT, false>(a, vec, idxb, grid, lds, s);
}

template <int Q>
hipError_t launch_fwd_out(const FwdArgs &a, int out, int vec, int idxb, dim3 grid, size_t lds, hipStream_t s) {
    switch (out) {
        case PLE_DTYPE_F32: return launch_fwd_bias<Q, PLE_DTYPE_F32>(a, vec, idxb, grid, lds, s);
        case PLE_DTYPE_F16: return launch_fwd_bias<Q, PLE_DTYPE_F16>(a, vec, idxb, grid, lds, s);
        default: return launch_fwd_bias<Q, PLE_DTYPE_BF16>(a, vec, idxb, grid, lds, s);
    }
}

struct BwdPlan {
    int C;
    int64_t NC;
    size_t part_bytes, part_db_bytes, tot_bytes;
    size_t total() const;
};

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

size_t BwdPlan::total() const {
    return align_up(part_bytes, 256) + align_up(part_db_bytes, 256) + align_up(tot_bytes, 256);
}

constexpr size_t kPartialBudget = 64ull << 20;   // bytes of chunk partials

BwdPlan plan_backward(int64_t N, int64_t F, int64_t B, int64_t D) {
    BwdPlan pl;
    const int64_t waves = 32 * static_cast<int64_t>(device_cu_count());   // histogram waves in flight
    int64_t c = (waves + F - 1) / F;
    const int64_t per_chunk = F * B * 2 * D * static_cast<int64_t>(sizeof(float));
    const int64_t budget_c = static_cast<int64_t>(kPartialBudget) / (per_chunk > 0 ? per_chunk : 1);
    if (c > budget_c) c = budget_c;
    if (c > 1024) c = 1024;
    const int64_t max_c = (N + 63) / 64;  // at least 64 samples per chunk
    if (c > max_c) c = max_c;
    if (c < 1) c = 1;
    pl.NC = (N + c - 1) / c;
    if (pl.NC < 1) pl.NC = 1;
    pl.C = static_cast<int>((N + pl.NC - 1) / pl.NC);
    if (pl.C < 1) pl.C = 1;
    pl.part_bytes = static_cast<size_t>(pl.C) * F * B * 2 * D * sizeof(float);
    pl.part_db_bytes = static_cast<size_t>(pl.C) * F * D * sizeof(float);
    pl.tot_bytes = static_cast<size_t>(F) * B * 2 * D * sizeof(float);
    return pl;
}

template <int GD, int Q>
hipError_t launch_bwd_typed(BwdArgs a, int idxb, bool want_dx, bool want_dwdb, const BwdPlan &pl, hipStream_t s) {
    if (want_dx) {
        const int64_t pairs = a.N * a.F;
        int64_t blocks = (pairs + (kBlock / 16) - 1) / (kBlock / 16);
        const int64_t cap = static_cast<int64_t>(device_cu_count()) * 16;
        if (blocks > cap) blocks = cap;
        if (blocks < 1) blocks = 1;
        switch (idxb) {
            case 1: hipLaunchKernelGGL((ple_bwd_dx_kernel<GD, Q, uint8_t>), dim3(blocks), dim3(kBlock), 0, s, a); break;
            case 2: hipLaunchKernelGGL((ple_bwd_dx_kernel<GD, Q, int16_t>), dim3(blocks), dim3(kBlock), 0, s, a); break;
            default: hipLaunchKernelGGL((ple_bwd_dx_kernel<GD, Q, int32_t>), dim3(blocks), dim3(kBlock), 0, s, a); break;
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (want_dwdb) {
        const size_t lds = static_cast<size_t>(a.B) * a.D * 2 * sizeof(float);
        const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.F) * pl.C));
        switch (idxb) {
            case 1: hipLaunchKernelGGL((ple_bwd_hist_kernel<GD, Q, uint8_t>), grid, dim3(kWave), lds, s, a); break;
            case 2: hipLaunchKernelGGL((ple_bwd_hist_kernel<GD, Q, int16_t>), grid, dim3(kWave), lds, s, a); break;
            default: hipLaunchKernelGGL((ple_bwd_hist_kernel<GD, Q, int32_t>), grid, dim3(kWave), lds, s, a); break;
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const int64_t cells = static_cast<int64_t>(a.F) * a.B * 2 * a.D;
        hipLaunchKernelGGL(ple_bwd_reduce_chunks_kernel, dim3((cells + kBlock - 1) / kBlock), dim3(kBlock), 0, s, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        const int64_t cols = static_cast<int64_t>(a.F) * a.D;
        hipLaunchKernelGGL(ple_bwd_finalize_kernel, dim3((cols + kBlock - 1) / kBlock), dim3(kBlock), 0, s, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <int GD>
hipError_t launch_bwd_q(const BwdArgs &a, int q, int idxb, bool want_dx, bool want_dwdb, const BwdPlan &pl, hipStream_t s) {
    switch (q) {
        case PLE_DTYPE_F32: return launch_bwd_typed<GD, PLE_DTYPE_F32>(a, idxb, want_dx, want_dwdb, pl, s);
        case PLE_DTYPE_F16: return launch_bwd_typed<GD, PLE_DTYPE_F16>(a, idxb, want_dx, want_dwdb, pl, s);
        default: return launch_bwd_typed<GD, PLE_DTYPE_BF16>(a, idxb, want_dx, want_dwdb, pl, s);
    }
}

int check_common(int64_t N, int64_t F, int64_t B, int64_t D) {
    if (N < 0 || F < 1 || B < 1 || D < 1) return PLE_E_BAD_SHAPE;
    if (F > INT32_MAX / 2 || B > INT32_MAX / 4 || D > 64) return PLE_E_TOO_LARGE;
    if (N > INT64_MAX / (F * D)) return PLE_E_TOO_LARGE;
    return PLE_OK;
}

}  // namespace

extern "C" {

int ple_abi_version(void) { return (1 << 16) | 0; }

int ple_bin_index_bytes(int64_t max_n_bins) { return idx_bytes_for(max_n_bins); }

const char *ple_error_string(int code) {
    switch (code) {
        case PLE_OK: return "success";
        case PLE_E_NULL_POINTER: return "a required pointer is NULL";
        case PLE_E_BAD_SHAPE: return "invalid shape (need N >= 0 and F, B, D >= 1)";
        case PLE_E_BAD_DTYPE: return "invalid dtype code";
        case PLE_E_BAD_INDEX_WIDTH: return "invalid bin index width";
        case PLE_E_TOO_LARGE: return "sizes exceed the supported range (D <= 64, F*B*D fits the kernels' index types)";
        case PLE_E_WORKSPACE: return "workspace is NULL, too small or not 256-byte aligned";
        case PLE_E_UNSUPPORTED: return "shape not supported by the LDS-resident kernels (per-feature tables exceed LDS)";
        case PLE_E_MISALIGNED: return "pointer misaligned for its element type";
        default: break;
    }
    if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
    return "unknown error";
}

int ple_forward_launch(const float *x, const float *bin_edges, const float *inv_bin_widths,
                       const int32_t *n_bins, const float *weight, const float *bias,
                       void *output, void *bin_indices, int64_t N, int64_t F, int64_t B,
                       int64_t D, int quant_dtype, int output_dtype, void *stream) {
    int rc = check_common(N, F, B, D);
    if (rc != PLE_OK) return rc;
    if (!valid_dtype(quant_dtype) || !valid_dtype(output_dtype)) return PLE_E_BAD_DTYPE;
    if (N == 0) return PLE_OK;
    if (!x || !bin_edges || !inv_bin_widths || !n_bins || !weight || !output || !bin_indices)
        return PLE_E_NULL_POINTER;
    const int out_bytes = output_dtype == PLE_DTYPE_F32 ? 4 : 2;
    const bool aligned16 = (reinterpret_cast<uintptr_t>(output) % (4 * out_bytes) == 0) &&
                           (reinterpret_cast<uintptr_t>(weight) % 16 == 0);
    if (reinterpret_cast<uintptr_t>(output) % out_bytes != 0) return PLE_E_MISALIGNED;
    FwdPlan pl;
    if (!plan_forward(N, F, B, D, aligned16, pl)) return PLE_E_UNSUPPORTED;
    FwdArgs a;
    a.x = x; a.edges = bin_edges; a.iw = inv_bin_widths; a.nbins = n_bins; a.weight = weight;
    a.bias = bias; a.out = output; a.idx = bin_indices;
    a.N = N; a.F = static_cast<int>(F); a.B = static_cast<int>(B); a.D = static_cast<int>(D);
    a.FS = pl.FS; a.G = pl.G; a.C = pl.C; a.NC = pl.NC;
    const int64_t grid = static_cast<int64_t>(pl.G) * pl.C;
    if (grid > INT32_MAX) return PLE_E_TOO_LARGE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int idxb = idx_bytes_for(B);
    hipError_t e;
    switch (quant_dtype) {
        case PLE_DTYPE_F32: e = launch_fwd_out<PLE_DTYPE_F32>(a, output_dtype, pl.vec, idxb, dim3(grid), pl.lds, s); break;
        case PLE_DTYPE_F16: e = launch_fwd_out<PLE_DTYPE_F16>(a, output_dtype, pl.vec, idxb, dim3(grid), pl.lds, s); break;
        default: e = launch_fwd_out<PLE_DTYPE_BF16>(a, output_dtype, pl.vec, idxb, dim3(grid), pl.lds, s); break;
    }
    return e == hipSuccess ? PLE_OK : static_cast<int>(e);
}

size_t ple_backward_workspace_bytes(int64_t N, int64_t F, int64_t B, int64_t D) {
    if (check_common(N, F, B, D) != PLE_OK || N == 0) return 0;
    return plan_backward(N, F, B, D).total();
}

int ple_backward_launch(const void *grad_output, const float *x, const float *bin_edges,
                        const float *inv_bin_widths, const int32_t *n_bins,
                        const float *weight, const void *bin_indices, float *grad_x,
                        float *grad_weight, float *grad_bias, int64_t N, int64_t F,
                        int64_t B, int64_t D, int grad_dtype, int quant_dtype,
                        void *workspace, size_t workspace_bytes, void *stream) {
    int rc = check_common(N, F, B, D);
    if (rc != PLE_OK) return rc;
    if (!valid_dtype(grad_dtype) || !valid_dtype(quant_dtype)) return PLE_E_BAD_DTYPE;
    const bool want_dx = grad_x != nullptr;
    const bool want_dwdb = grad_weight != nullptr || grad_bias != nullptr;
    if (!want_dx && !want_dwdb) return PLE_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (N == 0) {
        // empty batch: gradients of the parameters are zero
        hipError_t e = hipSuccess;
        if (grad_weight) e = hipMemsetAsync(grad_weight, 0, sizeof(float) * F * B * D, s);
        if (e == hipSuccess && grad_bias) e = hipMemsetAsync(grad_bias, 0, sizeof(float) * F * D, s);
        return e == hipSuccess ? PLE_OK : static_cast<int>(e);
    }
    if (!grad_output || !x || !bin_edges || !inv_bin_widths || !n_bins || !weight || !bin_indices)
        return PLE_E_NULL_POINTER;
    const size_t lds = static_cast<size_t>(B) * D * 2 * sizeof(float);
    if (want_dwdb && lds > kLdsMax) return PLE_E_UNSUPPORTED;
    BwdPlan pl = plan_backward(N, F, B, D);
    const size_t need = pl.total();
    if (want_dwdb && (workspace == nullptr || workspace_bytes < need ||
                      reinterpret_cast<uintptr_t>(workspace) % 256 != 0))
        return PLE_E_WORKSPACE;
    if (static_cast<int64_t>(F) * pl.C > INT32_MAX) return PLE_E_TOO_LARGE;
    BwdArgs a;
    a.g = grad_output; a.x = x; a.edges = bin_edges; a.iw = inv_bin_widths; a.nbins = n_bins;
    a.weight = weight; a.idx = bin_indices; a.dx = grad_x; a.dw = grad_weight; a.db = grad_bias;
    a.part = static_cast<float *>(workspace);
    char *ws = static_cast<char *>(workspace);
    a.part_db = want_dwdb ? reinterpret_cast<float *>(ws + align_up(pl.part_bytes, 256)) : nullptr;
    a.tot = want_dwdb ? reinterpret_cast<float *>(ws + align_up(pl.part_bytes, 256) + align_up(pl.part_db_bytes, 256))
                      : nullptr;
    a.N = N; a.F = static_cast<int>(F); a.B = static_cast<int>(B); a.D = static_cast<int>(D);
    a.C = pl.C; a.NC = pl.NC;
    const int idxb = idx_bytes_for(B);
    hipError_t e;
    switch (grad_dtype) {
        case PLE_DTYPE_F32: e = launch_bwd_q<PLE_DTYPE_F32>(a, quant_dtype, idxb, want_dx, want_dwdb, pl, s); break;
        case PLE_DTYPE_F16: e = launch_bwd_q<PLE_DTYPE_F16>(a, quant_dtype, idxb, want_dx, want_dwdb, pl, s); break;
        default: e = launch_bwd_q<PLE_DTYPE_BF16>(a, quant_dtype, idxb, want_dx, want_dwdb, pl, s); break;
    }
    return e == hipSuccess ? PLE_OK : static_cast<int>(e);
}

}  // extern "C"
