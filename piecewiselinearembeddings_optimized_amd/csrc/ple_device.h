// Device-side helpers shared by the PLE kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <stddef.h>
#include <stdint.h>

#include "../../include/ple_hip.h"

namespace ple {

constexpr int kWave = 64;
constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kNumXcd = 8;

// ---------------------------------------------------------------------------
// element conversions
// ---------------------------------------------------------------------------

// float -> bfloat16, nearest-even, by gfx950's conversion instruction
// (v_cvt_pk_bf16_f32, two values a dword: `lo` in bits 0-15, `hi` in bits
// 16-31).  For every fp32 input that is not a NaN it gives the bits of the
// integer formulation (u + 0x7fff + ((u >> 16) & 1)) >> 16 -- checked on an
// MI355X over all 2^32 input patterns, denormals and infinities included; a
// NaN stays a quiet NaN, keeping its sign and top payload bits (where the
// integer formulation returns 0x7fc0).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t bf16_pack2(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// float -> bfloat16 -> float (one instruction: the rounded value lands in the
// high half, above a zero low half)
__device__ __forceinline__ float bf16_round(float v) { return __uint_as_float(bf16_pack2(0.0f, v)); }

__device__ __forceinline__ uint16_t bf16_bits(float v) { return static_cast<uint16_t>(bf16_pack2(v, 0.0f)); }

// float -> IEEE half (nearest-even).  The empty asm pins v as an fp32 value:
// without it the compiler may fuse the multiply or fma that produced v with
// the conversion (v_fma_mix*_f16), rounding once to half instead of first to
// fp32 and then to half as the reference arithmetic does.
__device__ __forceinline__ float f16_round(float v) {
    __asm__ volatile("" : "+v"(v));
    return static_cast<float>(static_cast<_Float16>(v));
}

__device__ __forceinline__ uint16_t f16_bits(float v) {
    __asm__ volatile("" : "+v"(v));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// Round trip through the quantisation dtype (identity for fp32).
template <int Q>
__device__ __forceinline__ float quant(float v) {
    if constexpr (Q == PLE_DTYPE_BF16) return bf16_round(v);
    else if constexpr (Q == PLE_DTYPE_F16) return f16_round(v);
    else return v;
}

__device__ __forceinline__ float bf16_to_float(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ float f16_to_float(uint16_t b) {
    return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

template <int G>
__device__ __forceinline__ float load_grad(const void *p, int64_t i) {
    if constexpr (G == PLE_DTYPE_F32) return static_cast<const float *>(p)[i];
    else if constexpr (G == PLE_DTYPE_BF16) return bf16_to_float(static_cast<const uint16_t *>(p)[i]);
    else return f16_to_float(static_cast<const uint16_t *>(p)[i]);
}

// Loads VEC consecutive gradient elements starting at element i (i is a
// multiple of VEC; the base is aligned for the vector width).  VEC in
// {1, 2, 4, 8}.
template <int G, int VEC>
__device__ __forceinline__ void load_grad_vec(const void *p, int64_t i, float *out) {
    if constexpr (G == PLE_DTYPE_F32) {
        const float *q = static_cast<const float *>(p) + i;
        if constexpr (VEC == 8) {
            const float4 v0 = reinterpret_cast<const float4 *>(q)[0];
            const float4 v1 = reinterpret_cast<const float4 *>(q)[1];
            out[0] = v0.x; out[1] = v0.y; out[2] = v0.z; out[3] = v0.w;
            out[4] = v1.x; out[5] = v1.y; out[6] = v1.z; out[7] = v1.w;
        } else if constexpr (VEC == 4) {
            const float4 v = *reinterpret_cast<const float4 *>(q);
            out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
        } else if constexpr (VEC == 2) {
            const float2 v = *reinterpret_cast<const float2 *>(q);
            out[0] = v.x; out[1] = v.y;
        } else {
            out[0] = q[0];
        }
    } else {
        const uint16_t *q = static_cast<const uint16_t *>(p) + i;
        uint16_t h[VEC];
        if constexpr (VEC == 8) {
            const uint4 v = *reinterpret_cast<const uint4 *>(q);
            h[0] = v.x & 0xffffu; h[1] = v.x >> 16; h[2] = v.y & 0xffffu; h[3] = v.y >> 16;
            h[4] = v.z & 0xffffu; h[5] = v.z >> 16; h[6] = v.w & 0xffffu; h[7] = v.w >> 16;
        } else if constexpr (VEC == 4) {
            const uint2 v = *reinterpret_cast<const uint2 *>(q);
            h[0] = v.x & 0xffffu; h[1] = v.x >> 16; h[2] = v.y & 0xffffu; h[3] = v.y >> 16;
        } else if constexpr (VEC == 2) {
            const uint32_t v = *reinterpret_cast<const uint32_t *>(q);
            h[0] = v & 0xffffu; h[1] = v >> 16;
        } else {
            h[0] = q[0];
        }
#pragma unroll
        for (int t = 0; t < VEC; ++t)
            out[t] = (G == PLE_DTYPE_BF16) ? bf16_to_float(h[t]) : f16_to_float(h[t]);
    }
}

// Buffer resource over `bytes` bytes at `base` (raw addressing, stride 0).
// Loads at byte offsets at or beyond `bytes` return zeros.  Both arguments
// must be wave-uniform; they pass through readfirstlane so the compiler
// keeps the resource in scalar registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32));
    void *pu = reinterpret_cast<void *>((static_cast<uint64_t>(hi) << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(pu, static_cast<short>(0),
                                             static_cast<int>(__builtin_amdgcn_readfirstlane(bytes)), 0x00020000);
}

// Cache-policy operand of the buffer / global memory builtins: the
// non-temporal (streaming) hint.  Data read or written once -- the forward's
// output, gradient rows that fill whole 128-byte lines -- moves through the
// caches without displacing lines that are reused.
constexpr int kCpolNT = 2;

// VEC consecutive gradient elements at byte offset `off` of a buffer
// resource, as floats (VEC in {1, 2, 4, 8}; `off` aligned for the access);
// CPOL: cache-policy bits of the loads.
template <int G, int VEC, int CPOL = 0>
__device__ __forceinline__ void load_grad_buf(__amdgpu_buffer_rsrc_t rs, uint32_t off, float *out) {
    if constexpr (G == PLE_DTYPE_F32) {
        if constexpr (VEC >= 4) {
#pragma unroll
            for (int q = 0; q < VEC / 4; ++q) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * q, 0, CPOL);
                out[4 * q] = __uint_as_float(v[0]); out[4 * q + 1] = __uint_as_float(v[1]);
                out[4 * q + 2] = __uint_as_float(v[2]); out[4 * q + 3] = __uint_as_float(v[3]);
            }
        } else if constexpr (VEC == 2) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, CPOL);
            out[0] = __uint_as_float(v[0]); out[1] = __uint_as_float(v[1]);
        } else {
            out[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, CPOL));
        }
    } else {
        uint32_t w[VEC / 2 > 0 ? VEC / 2 : 1];
        if constexpr (VEC == 8) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, CPOL);
            w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
        } else if constexpr (VEC == 4) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, CPOL);
            w[0] = v[0]; w[1] = v[1];
        } else if constexpr (VEC == 2) {
            w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, CPOL);
        } else {
            w[0] = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, CPOL);
        }
#pragma unroll
        for (int t = 0; t < VEC; ++t) {
            const uint16_t h = static_cast<uint16_t>(w[t / 2] >> (16 * (t % 2)));
            out[t] = (G == PLE_DTYPE_BF16) ? bf16_to_float(h) : f16_to_float(h);
        }
    }
}

// Dwords a lane holds for VEC gradient elements of a row: one per element for
// fp32, two elements each for the 16-bit types, kept as loaded and widened at
// use (grad_elem), so a 16-bit row costs half the registers of its floats.
template <int G, int VEC>
constexpr int grad_words() {
    return G == PLE_DTYPE_F32 ? VEC : (VEC + 1) / 2;
}

template <int G, int VEC, int CPOL = 0>
__device__ __forceinline__ void load_grad_words(__amdgpu_buffer_rsrc_t rs, uint32_t off,
                                                uint32_t (&w)[grad_words<G, VEC>()]) {
    constexpr int W = grad_words<G, VEC>();
    if constexpr (W % 4 == 0) {
#pragma unroll
        for (int q = 0; q < W / 4; ++q) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * q, 0, CPOL);
            w[4 * q] = v[0]; w[4 * q + 1] = v[1]; w[4 * q + 2] = v[2]; w[4 * q + 3] = v[3];
        }
    } else if constexpr (W == 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, CPOL);
        w[0] = v[0]; w[1] = v[1];
    } else if constexpr (G == PLE_DTYPE_F32 || VEC == 2) {
        w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, CPOL);
    } else {
        w[0] = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, CPOL);   // (low half)
    }
}

// Element q (a compile-time index) of a row held as load_grad_words left it.
template <int G>
__device__ __forceinline__ float grad_elem(const uint32_t *w, int q) {
    if constexpr (G == PLE_DTYPE_F32) {
        return __uint_as_float(w[q]);
    } else {
        const uint32_t x = w[q >> 1];
        if constexpr (G == PLE_DTYPE_BF16) return __uint_as_float((q & 1) ? (x & 0xffff0000u) : (x << 16));
        else return f16_to_float(static_cast<uint16_t>((q & 1) ? (x >> 16) : x));
    }
}

// VEC consecutive floats from / to LDS (16-byte accesses for VEC 4 and 8,
// 8-byte for VEC 2; the address is aligned to the access in those cases).
template <int VEC>
__device__ __forceinline__ void lds_load_vec(const float *p, float *v) {
    if constexpr (VEC % 4 == 0) {
#pragma unroll
        for (int q = 0; q < VEC / 4; ++q) {
            const float4 t = reinterpret_cast<const float4 *>(p)[q];
            v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
        }
    } else if constexpr (VEC == 2) {
        const float2 t = *reinterpret_cast<const float2 *>(p);
        v[0] = t.x; v[1] = t.y;
    } else {
#pragma unroll
        for (int t = 0; t < VEC; ++t) v[t] = p[t];
    }
}

template <int VEC>
__device__ __forceinline__ void lds_store_vec(float *p, const float *v) {
    if constexpr (VEC % 4 == 0) {
#pragma unroll
        for (int q = 0; q < VEC / 4; ++q)
            reinterpret_cast<float4 *>(p)[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    } else if constexpr (VEC == 2) {
        *reinterpret_cast<float2 *>(p) = make_float2(v[0], v[1]);
    } else {
#pragma unroll
        for (int t = 0; t < VEC; ++t) p[t] = v[t];
    }
}

// Two outputs rounded to a 16-bit OUT, packed into a dword (a in the low half).
template <int OUT>
__device__ __forceinline__ uint32_t pack16(float a, float b) {
    if constexpr (OUT == PLE_DTYPE_BF16) return bf16_pack2(a, b);
    else return static_cast<uint32_t>(f16_bits(a)) | (static_cast<uint32_t>(f16_bits(b)) << 16);
}

// Stores VEC consecutive outputs as OUT (VEC in {1, 2, 4}; 8 for 16-bit OUT).
// Four or more outputs a lane, and pairs of 16-bit outputs, are stored with
// the non-temporal hint when `nt` (the output is written once and not read
// back here); one or two fp32 outputs and single 16-bit outputs (rows of D not
// a multiple of 4, resp. odd D) are plain stores, since with the hint they
// measured up to 40% slower (F=128, 48 bins, N=65536: d=30 fp32 456 -> 321 us,
// d=31 484 -> 340 us, d=15 bf16 188 -> 165 us without it; pairs of bf16 at
// d=30 were about even).  NT = false: every store plain.  (A compile-time
// choice: with a run-time one the compiler merges the two stores into one
// without the hint.)
template <int OUT, int VEC, bool NT = true>
__device__ __forceinline__ void store_out(void *base, int64_t i, const float *v) {
    constexpr bool nt = NT;
    if constexpr (OUT == PLE_DTYPE_F32) {
        float *p = static_cast<float *>(base) + i;
        if constexpr (VEC == 4) {
            typedef float f32x4 __attribute__((ext_vector_type(4)));
            const f32x4 t = {v[0], v[1], v[2], v[3]};
            if constexpr (nt) __builtin_nontemporal_store(t, reinterpret_cast<f32x4 *>(p));
            else *reinterpret_cast<f32x4 *>(p) = t;
        } else if constexpr (VEC == 2) {
            *reinterpret_cast<float2 *>(p) = make_float2(v[0], v[1]);
        } else {
            p[0] = v[0];
        }
    } else {
        uint16_t *p = static_cast<uint16_t *>(base) + i;
        if constexpr (VEC == 8) {
            typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
            const u32x4 w = {pack16<OUT>(v[0], v[1]), pack16<OUT>(v[2], v[3]), pack16<OUT>(v[4], v[5]),
                             pack16<OUT>(v[6], v[7])};
            if constexpr (nt) __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(p));
            else *reinterpret_cast<u32x4 *>(p) = w;
        } else if constexpr (VEC == 4) {
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            const u32x2 w = {pack16<OUT>(v[0], v[1]), pack16<OUT>(v[2], v[3])};
            if constexpr (nt) __builtin_nontemporal_store(w, reinterpret_cast<u32x2 *>(p));
            else *reinterpret_cast<u32x2 *>(p) = w;
        } else if constexpr (VEC == 2) {
            if constexpr (nt) __builtin_nontemporal_store(pack16<OUT>(v[0], v[1]), reinterpret_cast<uint32_t *>(p));
            else *reinterpret_cast<uint32_t *>(p) = pack16<OUT>(v[0], v[1]);
        } else {
            p[0] = OUT == PLE_DTYPE_BF16 ? bf16_bits(v[0]) : f16_bits(v[0]);
        }
    }
}

// ---------------------------------------------------------------------------
// lane-group reductions
// ---------------------------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Lane i of each quad of lanes, to all four (quad_perm [i,i,i,i]); i must fold
// to a constant (an unrolled loop index).  All lanes of the quad must be active.
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v, int i) {
    const int s = static_cast<int>(v);
    switch (i) {
        case 0: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, s, 0x00, 0xF, 0xF, false));
        case 1: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, s, 0x55, 0xF, 0xF, false));
        case 2: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, s, 0xAA, 0xF, 0xF, false));
        default: return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, s, 0xFF, 0xF, 0xF, false));
    }
}

// Sum over aligned groups of W lanes (W a power of two); every lane of the
// group receives the sum.  Groups of up to 16 lanes reduce with DPP inside a
// 16-lane row (quad permutes, then half-row and row mirrors); wider groups
// finish with cross-row shuffles.  All lanes of a group must be active.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "group width must be a power of two");
    if constexpr (W >= 2) v += dpp_f32<0xB1>(v);    // quad_perm [1,0,3,2]
    if constexpr (W >= 4) v += dpp_f32<0x4E>(v);    // quad_perm [2,3,0,1]
    if constexpr (W >= 8) v += dpp_f32<0x141>(v);   // row_half_mirror
    if constexpr (W >= 16) v += dpp_f32<0x140>(v);  // row_mirror
    if constexpr (W >= 32) v += __shfl_xor(v, 16);
    if constexpr (W >= 64) v += __shfl_xor(v, 32);
    return v;
}

// Reduce-scatter of four values per lane over aligned groups of W lanes
// (W in {4, 8, 16}): returns the group sum of p[r] with r = the lane's row,
// r = 2 * bit(log2 W - 1) + bit(log2 W - 2) of its index in the group.  Each
// step exchanges half of what a lane still holds with a partner that differs
// in one bit -- the partners are XOR masks (mirrors are XOR 15 / XOR 7), so
// the four steps cover the group exactly once.
template <int W>
__device__ __forceinline__ float group_reduce_scatter4(const float (&p)[4], int lc) {
    static_assert(W == 4 || W == 8 || W == 16, "group width");
    constexpr int LOG = W == 4 ? 2 : (W == 8 ? 3 : 4);
    // DPP controls by the bit a partner differs in
    constexpr int kCtrl[4] = {0xB1, 0x4E, 0x141, 0x140};   // xor 1, xor 2, xor 7 (half-row mirror), xor 15 (row mirror)
    const bool hi_a = (lc >> (LOG - 1)) & 1;
    float k0 = hi_a ? p[2] : p[0];
    float k1 = hi_a ? p[3] : p[1];
    const float s0 = hi_a ? p[0] : p[2];
    const float s1 = hi_a ? p[1] : p[3];
    k0 += dpp_f32<kCtrl[LOG - 1]>(s0);
    k1 += dpp_f32<kCtrl[LOG - 1]>(s1);
    const bool hi_b = (lc >> (LOG - 2)) & 1;
    float k = hi_b ? k1 : k0;
    k += dpp_f32<kCtrl[LOG - 2]>(hi_b ? k0 : k1);
    if constexpr (LOG >= 4) k += dpp_f32<kCtrl[1]>(k);
    if constexpr (LOG >= 3) k += dpp_f32<kCtrl[0]>(k);
    return k;
}

// Same, for a group width known only at run time (power of two <= 64).
__device__ __forceinline__ float group_sum_rt(float v, int w) {
    for (int off = w >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, w);
    return v;
}

// ---------------------------------------------------------------------------
// bins
// ---------------------------------------------------------------------------

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

// The last real bin's parameters live in slot bmax-1.
__host__ __device__ __forceinline__ int phys_bin(int k, int n, int bmax) {
    return k == n - 1 ? bmax - 1 : k;
}

template <typename IdxT>
__device__ __forceinline__ int load_idx(const void *p, int64_t i) {
    return static_cast<int>(static_cast<const IdxT *>(p)[i]);
}

// Workgroup -> (feature group g, sample chunk c), XCD aware.  Workgroup ids
// are dealt to the XCDs round-robin; tiles are numbered chunk-major
// (t = c * G + g) and each XCD takes one contiguous run of tiles.  The feature
// groups of a chunk, which share that chunk's cache lines of x, of the bin
// indices and of dx, therefore run on one XCD and share its L2; with fewer
// chunks than XCDs a chunk's feature range is split between XCDs instead of
// piling onto one.  The grid is kNumXcd * tiles_per_xcd(G, C) workgroups.
__host__ __device__ __forceinline__ int64_t tiles_per_xcd(int64_t G, int64_t C) {
    return (G * C + kNumXcd - 1) / kNumXcd;
}

__device__ __forceinline__ bool decode_tile(int bid, int G, int C, int &g, int &c) {
    const int x8 = bid % kNumXcd;
    const int64_t L = bid / kNumXcd;
    const int64_t tpx = tiles_per_xcd(G, C);
    const int64_t t = x8 * tpx + L;
    if (L >= tpx || t >= static_cast<int64_t>(G) * C) return false;
    c = static_cast<int>(t / G);
    g = static_cast<int>(t - static_cast<int64_t>(c) * G);
    return true;
}

}  // namespace ple
