// Dense piecewise-linear encoding (gfx950): the output of the upstream
// PiecewiseLinearEncoding module (rtdl_num_embeddings==0.0.12), restated.
//
// For feature f with n_f bins, bin b = the clamped right-sided search of x
// (as in the fused embedding) and frac = (x - e_b) * iw_b, the n_f
// components written at columns off_f .. off_f + n_f - 1 of the output row are
//     component k = 1 (k < b),  frac (k == b),  0 (k > b)
// which is upstream's clamp pattern: middle bins clamped to [0, 1], the first
// bin only above, the last bin only below, a single bin not at all (the
// component k == b is exactly the one no clamp touches).  A NaN x gives NaN
// components (torch.clamp propagates NaN).
//
// Backward: dx = g[off_f + b] * iw_b, plus g[off_f + b - 1] * iw_{b-1} when
// b > 0 and x == e_b (both neighbouring clamps pass at their bounds) -- the
// same two-term rule as the embedding's dx.
//
// Forward kernel: one workgroup per block of kEncRows samples.  Phase 1
// computes (b, frac) of every (sample, feature) pair of the block into LDS;
// phase 2 walks the output row in 16-byte groups -- each thread finds the
// features of its columns once (binary search over the LDS column offsets)
// and then writes them for every sample of the block, so each store
// instruction covers 1 KiB of one row.

#include "ple_device.h"
#include "ple_internal.h"

namespace ple {
namespace {

constexpr int kEncRows = 8;   // samples per workgroup

struct EncArgs {
    const float *x, *edges, *iw;
    const int32_t *nbins, *offsets;
    const float *g;      // backward: grad_output [N, T]
    float *out;          // forward: [N, T]; backward: grad_x [N, F]
    int64_t N;
    int F, B, T;
};

__device__ __forceinline__ float enc_value(int k, int b, float frac) {
    // NaN x: every component NaN (frac is NaN exactly then)
    if (frac != frac) return frac;
    return k < b ? 1.0f : (k == b ? frac : 0.0f);
}

template <bool V4>
__global__ __launch_bounds__(kBlock) void ple_encode_kernel(EncArgs a) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int F = a.F, B = a.B, T = a.T;
    int *s_off = reinterpret_cast<int *>(lds);                 // [F + 1] column offsets
    int *s_bin = s_off + F + 1;                                // [kEncRows][F]
    float *s_frac = reinterpret_cast<float *>(s_bin + kEncRows * F);
    const int tid = threadIdx.x;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kEncRows;
    const int ns = static_cast<int>(min(static_cast<int64_t>(kEncRows), a.N - n0));

    for (int i = tid; i < F; i += kBlock) s_off[i] = a.offsets[i];
    if (tid == 0) s_off[F] = T;
    for (int i = tid; i < ns * F; i += kBlock) {
        const int s = i / F;
        const int f = i - s * F;
        const float v = a.x[(n0 + s) * F + f];
        const int n = clamp_nbins(a.nbins[f], B);
        const float *e = a.edges + static_cast<int64_t>(f) * (B + 1);
        const int b = find_bin(v, e, n);
        s_bin[i] = b;
        s_frac[i] = (v - e[b]) * a.iw[static_cast<int64_t>(f) * B + b];
    }
    __syncthreads();

    constexpr int W = V4 ? 4 : 1;
    for (int p0 = tid * W; p0 < T; p0 += kBlock * W) {
        // feature of column p0: last f with off[f] <= p0
        int lo = 0, hi = F;          // invariant: off[lo] <= p0 < off[hi]
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (s_off[mid] <= p0) lo = mid;
            else hi = mid;
        }
        int fq[W], kq[W];
        int f = lo;
#pragma unroll
        for (int j = 0; j < W; ++j) {
            const int p = min(p0 + j, T - 1);
            while (f + 1 < F && p >= s_off[f + 1]) ++f;
            fq[j] = f;
            kq[j] = p - s_off[f];
        }
        for (int s = 0; s < ns; ++s) {
            float v[W];
#pragma unroll
            for (int j = 0; j < W; ++j) v[j] = enc_value(kq[j], s_bin[s * F + fq[j]], s_frac[s * F + fq[j]]);
            store_out<PLE_DTYPE_F32, W>(a.out, (n0 + s) * T + p0, v);
        }
    }
}

// One thread per (sample, feature) pair.
__global__ __launch_bounds__(kBlock) void ple_encode_backward_kernel(EncArgs a) {
    const int F = a.F, B = a.B, T = a.T;
    const int64_t pairs = a.N * F;
    for (int64_t p = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; p < pairs;
         p += static_cast<int64_t>(gridDim.x) * kBlock) {
        const int64_t n = p / F;
        const int f = static_cast<int>(p - n * F);
        const float v = a.x[p];
        const int nb = clamp_nbins(a.nbins[f], B);
        const float *e = a.edges + static_cast<int64_t>(f) * (B + 1);
        const float *iw = a.iw + static_cast<int64_t>(f) * B;
        const int b = find_bin(v, e, nb);
        // column of component b; columns outside [0, T) (offsets that do not
        // match n_bins) read nothing
        const int c = a.offsets[f] + b;
        const float *grow = a.g + n * T;
        float r = (c >= 0 && c < T) ? grow[c] * iw[b] : 0.0f;
        if (b > 0 && v == e[b] && c - 1 >= 0 && c - 1 < T) r = fmaf(grow[c - 1], iw[b - 1], r);
        a.out[p] = r;
    }
}

size_t enc_lds_bytes(int F) {
    return sizeof(int) * (F + 1) + (sizeof(int) + sizeof(float)) * static_cast<size_t>(kEncRows) * F;
}

}  // namespace

int encode_run(const EncodeRequest &r) {
    if (r.T < 1 || r.T > INT32_MAX / 2) return PLE_E_TOO_LARGE;
    const size_t lds = enc_lds_bytes(static_cast<int>(r.F));
    if (lds > kLdsMax) return PLE_E_UNSUPPORTED;
    EncArgs a{};
    a.x = r.x; a.edges = r.edges; a.iw = r.iw; a.nbins = r.nbins; a.offsets = r.offsets;
    a.out = r.out;
    a.N = r.N; a.F = static_cast<int>(r.F); a.B = static_cast<int>(r.B); a.T = static_cast<int>(r.T);
    const int64_t blocks = (r.N + kEncRows - 1) / kEncRows;
    if (blocks > INT32_MAX) return PLE_E_TOO_LARGE;
    const bool v4 = r.T % 4 == 0 && reinterpret_cast<uintptr_t>(r.out) % 16 == 0;
    if (v4) hipLaunchKernelGGL(ple_encode_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), lds, r.stream, a);
    else hipLaunchKernelGGL(ple_encode_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), lds, r.stream, a);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? PLE_OK : static_cast<int>(e);
}

int encode_backward_run(const EncodeRequest &r) {
    if (r.T < 1 || r.T > INT32_MAX / 2) return PLE_E_TOO_LARGE;
    EncArgs a{};
    a.x = r.x; a.edges = r.edges; a.iw = r.iw; a.nbins = r.nbins; a.offsets = r.offsets;
    a.g = r.g; a.out = r.out;
    a.N = r.N; a.F = static_cast<int>(r.F); a.B = static_cast<int>(r.B); a.T = static_cast<int>(r.T);
    const int64_t pairs = r.N * r.F;
    int64_t blocks = (pairs + kBlock - 1) / kBlock;
    const int64_t cap = static_cast<int64_t>(device_cu_count()) * 32;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(ple_encode_backward_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, r.stream, a);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? PLE_OK : static_cast<int>(e);
}

}  // namespace ple
