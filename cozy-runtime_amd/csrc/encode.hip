// Weight encoders on gfx950: the producers of int8.convrot (rotation 256), fp8.rowwise, mxfp8,
// w4a8.convrot and nvfp4 weights from float32, bf16 or fp16 matrices, and the measure of what
// an encoding lost. The reference delegates these producers to tensorfs
// (derive/microscale.py:117-138,146-408: strategies int8-convrot256/1, fp8-rowwise-rne/1,
// w4a8-convrot256-fixed/1, nvfp4-min-sse/1), whose arithmetic is not in the reference; the laws
// here are this build's and each is restated in the CPU oracle:
// - int8.convrot: r = H256(w)·(1/16) in float32 in the reference's stage order, s = max(amax/127,
//   1e-12), q = clamp(rne(r/s), ±127) — the activation law (internal/int8_linear.py:422-428) on
//   weight rows, so encoding then decoding is the rotated int8 lane's own round trip.
// - fp8.rowwise: s = max(amax/448, 1e-12), q = e4m3(clamp(w/s, ±448)) (internal/probe.py:706-709).
// - mxfp8: the activation law per 32-block (internal/encoding/leaves.py:1411-1424), the E8M0 grid
//   row-major or in cuBLAS's 128x4 tiles.
// - w4a8.convrot: int8.convrot's r and s, t = r/s; per 16-group σ = e4m3(max|t| / max|c|) and each
//   code the nearest of the 16 levels clamp(rne(c[q]·σ), ±127) (first on a tie), c the codebook.
// - nvfp4: g = amax(|w|)/(448·6) (1 for an all-zero tensor); per 16-block the E4M3 scale among
//   e4m3(amax_b/(6g)) and its two neighbours with the least squared error of (e2m1·s)·g, codes
//   e2m1 of w/(s·g) rounded to nearest even and saturated at ±6.
// - svdq.int4g64 (this build's W4A4 variant): the residual w − up·down in float64 moved into the
//   smoothed basis, v = float32((w − up·down) / p); per 64-group s = fp16(amax|v| / 7), codes
//   clamp(rne(v / s), −8, 7) (0 where s == 0), two a byte with element 2k low.
#include "common.h"
#include "kernels.h"
#include "rotate.h"

namespace cozyq {
namespace {

constexpr int kEncThreads = 256;

// Eight consecutive elements of a float32 / bf16 / fp16 matrix from element `e` (8-aligned).
template <int kIn>
__device__ __forceinline__ void load8in(const void* x, int64_t e, float (&v)[8]) {
    if constexpr (kIn == kNumF32) {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + e);
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const uint4 raw = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + e);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = widen<kIn == kNumF16>(static_cast<uint16_t>(w[i] & 0xffffu));
            v[2 * i + 1] = widen<kIn == kNumF16>(static_cast<uint16_t>(w[i] >> 16));
        }
    }
}

template <int kIn>
__device__ __forceinline__ float load1in(const void* x, int64_t e) {
    if constexpr (kIn == kNumF32) return static_cast<const float*>(x)[e];
    else return widen<kIn == kNumF16>(static_cast<const uint16_t*>(x)[e]);
}

__device__ __forceinline__ float block_max_enc(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < kEncThreads / 64; ++i) m = fmaxf(m, red[i]);
    __syncthreads();
    return m;
}

// ------------------------------------------------------------ int8.convrot and w4a8.convrot

// One workgroup a row, K % 256 == 0. Two passes over the row's 4096-element chunks (the second
// from cache): the rotation and its amax, then the rotation again and the codes. Each thread's
// rotated values are one contiguous 16-run of a 256-group, which is one w4a8 group.
template <int kIn, bool kW4>
__global__ __launch_bounds__(kEncThreads) void encode_rotated_kernel(const void* __restrict__ w, int K,
                                                                     int8_t* __restrict__ q, float* __restrict__ scale,
                                                                     uint8_t* __restrict__ codes,
                                                                     uint8_t* __restrict__ group_scale,
                                                                     const float* __restrict__ codebook) {
    using L = Layout<256>;
    __shared__ __attribute__((aligned(16))) float lds[L::kFloats];
    __shared__ float red[kEncThreads / 64];
    const int row = blockIdx.x, tid = threadIdx.x;
    const void* wr = kIn == kNumF32 ? static_cast<const void*>(static_cast<const float*>(w) + static_cast<int64_t>(row) * K)
                                    : static_cast<const void*>(static_cast<const uint16_t*>(w) + static_cast<int64_t>(row) * K);
    const int chunks = (K + kChunk - 1) / kChunk;
    auto rotate = [&](int c, float (&out)[16], float& amax) {
        const int base = c * kChunk;
        const int width = min(kChunk, K - base);
        for (int e = tid * 8; e < width; e += kEncThreads * 8) {
            float v[8];
            load8in<kIn>(wr, base + e, v);
            const int g = e / 256, within = e % 256;
            float* dst = lds + L::at(g, within / 16, within % 16);
            *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            *reinterpret_cast<float4*>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
        }
        rotate_lds_chunk<256, kEncThreads>(lds, width, tid, out, amax);
        __syncthreads();
        return width / 256;
    };
    float amax = 0.0f;
    for (int c = 0; c < chunks; ++c) {
        float out[16];
        rotate(c, out, amax);
    }
    amax = block_max_enc(amax, red);
    const float s = fmaxf(amax / 127.0f, kScaleFloor);
    if (tid == 0) scale[row] = s;
    const float rs = 1.0f / s;
    const bool fast = s < __builtin_huge_valf();
    float levels_src[16], cmax = 0.0f;
    if constexpr (kW4) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            levels_src[k] = codebook[k];
            cmax = fmaxf(cmax, fabsf(levels_src[k]));
        }
    }
    for (int c = 0; c < chunks; ++c) {
        float out[16], unused = 0.0f;
        const int groups = rotate(c, out, unused);
        const int g = tid / L::kRuns, hi = tid % L::kRuns;
        if (g >= groups) continue;
        const int64_t at = static_cast<int64_t>(row) * K + c * kChunk + g * 256 + hi * 16;  // first element
        if constexpr (!kW4) {
            uint32_t packed[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t word = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int8_t b = fast ? q8<true>(out[4 * i + j], s, rs) : q8<false>(out[4 * i + j], s, rs);
                    word |= static_cast<uint32_t>(static_cast<uint8_t>(b)) << (8 * j);
                }
                packed[i] = word;
            }
            *reinterpret_cast<uint4*>(q + at) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
        } else {
            float t[16], ga = 0.0f;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                t[k] = fast ? div_rn(out[k], s, rs) : out[k] / s;
                ga = fmaxf(ga, fabsf(t[k]));
            }
            const uint32_t sb = e4m3_rn(fminf(ga / cmax, kE4m3Max));
            const float sigma = e4m3_value(sb);
            float lv[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const float p = levels_src[k] * sigma;
                lv[k] = p != p ? 0.0f : fminf(fmaxf(__builtin_rintf(p), -127.0f), 127.0f);
            }
            uint32_t packed[2] = {0, 0};
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                int best = 0;
                float err = fabsf(lv[0] - t[k]);
#pragma unroll
                for (int c2 = 1; c2 < 16; ++c2) {
                    const float e2 = fabsf(lv[c2] - t[k]);
                    if (e2 < err) { err = e2; best = c2; }
                }
                packed[k / 8] |= static_cast<uint32_t>(best) << (4 * (k % 8));
            }
            *reinterpret_cast<uint2*>(codes + at / 2) = make_uint2(packed[0], packed[1]);
            group_scale[at / 16] = static_cast<uint8_t>(sb);
        }
    }
}

// ------------------------------------------------------------------------- fp8.rowwise

template <int kIn>
__global__ __launch_bounds__(kEncThreads) void encode_fp8_rowwise_kernel(const void* __restrict__ w, int K,
                                                                         uint8_t* __restrict__ q,
                                                                         float* __restrict__ scale) {
    __shared__ float red[kEncThreads / 64];
    const int row = blockIdx.x, tid = threadIdx.x;
    const int64_t base = static_cast<int64_t>(row) * K;
    float amax = 0.0f;
    for (int e = tid * 8; e < K; e += kEncThreads * 8) {
        float v[8];
        load8in<kIn>(w, base + e, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    }
    amax = block_max_enc(amax, red);
    const float s = fmaxf(amax / kE4m3Max, kScaleFloor);
    if (tid == 0) scale[row] = s;
    const float rs = 1.0f / s;
    const bool fast = s < __builtin_huge_valf();
    for (int e = tid * 8; e < K; e += kEncThreads * 8) {
        float v[8], r[8];
        load8in<kIn>(w, base + e, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = fminf(fmaxf(fast ? div_rn(v[i], s, rs) : v[i] / s, -kE4m3Max), kE4m3Max);
        *reinterpret_cast<uint2*>(q + base + e) = make_uint2(e4m3x4(r[0], r[1], r[2], r[3]), e4m3x4(r[4], r[5], r[6], r[7]));
    }
}

// ------------------------------------------------------------------------------- mxfp8

// Four threads a 32-block, eight elements each (K % 32 == 0); the E8M0 byte lands row-major or
// at its 128x4 tile position.
template <int kIn>
__global__ __launch_bounds__(kEncThreads) void encode_mx_kernel(const void* __restrict__ w, int64_t rows, int K,
                                                                uint8_t* __restrict__ q, uint8_t* __restrict__ scale,
                                                                int tiled) {
    const int64_t total8 = rows * K / 8;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kEncThreads + threadIdx.x;
    const int64_t at = i < total8 ? i : total8 - 1;  // every lane takes part in the shuffles
    float v[8];
    load8in<kIn>(w, at * 8, v);
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(v[k]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    const uint32_t b = mx_byte(amax);
    // x / 2^(b-127) as x · 2^(127-b): the same real number, rounded once either way.
    const float inv = b >= 254 ? float_of(1u << 22) : float_of((254u - b) << 23);
    float r[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) r[k] = fminf(fmaxf(v[k] * inv, -kE4m3Max), kE4m3Max);
    if (i >= total8) return;
    *reinterpret_cast<uint2*>(q + at * 8) = make_uint2(e4m3x4(r[0], r[1], r[2], r[3]), e4m3x4(r[4], r[5], r[6], r[7]));
    if ((threadIdx.x & 3) == 0) {
        const int64_t row = at * 8 / K, blk = (at * 8 % K) / 32, width = K / 32;
        int64_t idx = row * width + blk;
        if (tiled)
            idx = ((row >> 7) * ((width + 3) >> 2) + (blk >> 2)) * 512 + (row & 31) * 16 + ((row & 127) >> 5) * 4 + (blk & 3);
        scale[idx] = static_cast<uint8_t>(b);
    }
}

// ------------------------------------------------------------------------------- nvfp4

// max |w| over the matrix into `amax` (float32 bits; the host zeroes it first). Non-negative
// floats order as their bit patterns, so an integer max is a float max.
template <int kIn>
__global__ __launch_bounds__(kEncThreads) void amax_kernel(const void* __restrict__ w, int64_t total,
                                                           uint32_t* __restrict__ amax) {
    __shared__ float red[kEncThreads / 64];
    float m = 0.0f;
    for (int64_t e = (static_cast<int64_t>(blockIdx.x) * kEncThreads + threadIdx.x) * 8; e < total;
         e += static_cast<int64_t>(gridDim.x) * kEncThreads * 8) {
        float v[8];
        load8in<kIn>(w, e, v);
#pragma unroll
        for (int k = 0; k < 8; ++k) m = fmaxf(m, fabsf(v[k]));
    }
    m = block_max_enc(m, red);
    if (threadIdx.x == 0) atomicMax(amax, bits_of(m));
}

// E2M1 code of x (nearest even on ties, saturated at ±6); bit 3 the sign of x.
__device__ __forceinline__ uint32_t e2m1_rn(float x) {
    const float a = fabsf(x);
    uint32_t m;
    if (a <= 0.25f) m = 0;
    else if (a < 0.75f) m = 1;
    else if (a <= 1.25f) m = 2;
    else if (a < 1.75f) m = 3;
    else if (a <= 2.5f) m = 4;
    else if (a < 3.5f) m = 5;
    else if (a <= 5.0f) m = 6;
    else m = 7;
    return (x < 0.0f ? 8u : 0u) | m;
}

__device__ __forceinline__ float e2m1_of(uint32_t nib) {
    const uint32_t m = nib & 7u, sign = (nib & 8u) << 28;
    const uint32_t mag = m < 2 ? (m ? 0x3f000000u : 0u) : (((m >> 1) + 126u) << 23) | ((m & 1u) << 22);
    return float_of(sign | mag);
}

// One thread a 16-block (K % 16 == 0): candidates e4m3(amax_b/(6g)) − 1, + 0, + 1 (positive
// codes), the one with the least squared error of (e2m1·s)·g kept, first of equals in the
// order (+0, −1, +1). `saturated` counts elements with |w/(s·g)| > 6.
template <int kIn>
__global__ __launch_bounds__(kEncThreads) void encode_nvfp4_kernel(const void* __restrict__ w, int64_t blocks,
                                                                   const uint32_t* __restrict__ amax_bits,
                                                                   uint8_t* __restrict__ codes,
                                                                   uint8_t* __restrict__ scale,
                                                                   float* __restrict__ scale_2,
                                                                   unsigned long long* __restrict__ saturated) {
    const int64_t b = static_cast<int64_t>(blockIdx.x) * kEncThreads + threadIdx.x;
    const float amax_t = float_of(*amax_bits);
    const float g = amax_t > 0.0f ? amax_t / (kE4m3Max * 6.0f) : 1.0f;
    if (b == 0) scale_2[0] = g;
    if (b >= blocks) return;
    float x[16];
    load8in<kIn>(w, b * 16, *reinterpret_cast<float(*)[8]>(x));
    load8in<kIn>(w, b * 16 + 8, *reinterpret_cast<float(*)[8]>(x + 8));
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) amax = fmaxf(amax, fabsf(x[k]));
    const uint32_t c0 = e4m3_rn(fminf(amax / (6.0f * g), kE4m3Max));
    const uint32_t cands[3] = {c0, c0 > 1 ? c0 - 1 : c0, c0 < 0x7e ? c0 + 1 : c0};
    uint32_t best = c0;
    float best_err = __builtin_huge_valf();
    for (int ci = 0; ci < 3; ++ci) {
        const uint32_t c = cands[ci];
        const float s = e4m3_value(c);
        const float d = s * g;
        float err = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float value = d > 0.0f ? (e2m1_of(e2m1_rn(x[k] / d)) * s) * g : 0.0f;
            const float diff = x[k] - value;
            err = err + diff * diff;
        }
        if (err < best_err) { best_err = err; best = c; }
    }
    const float s = e4m3_value(best), d = s * g;
    uint32_t packed[2] = {0, 0};
    unsigned long long sat = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float r = d > 0.0f ? x[k] / d : 0.0f;
        sat += fabsf(r) > 6.0f;
        packed[k / 8] |= e2m1_rn(r) << (4 * (k % 8));
    }
    *reinterpret_cast<uint2*>(codes + b * 8) = make_uint2(packed[0], packed[1]);
    scale[b] = static_cast<uint8_t>(best);
    if (sat) atomicAdd(saturated, sat);
}

// ------------------------------------------------------------------------ svdq.int4g64

// One thread an 8-element chunk (K % 64 == 0, so eight threads a group, in one wave): the
// residual in float64 (bf16 products are exact there; the sums are exact for all but extreme
// exponent spreads), divided by p in float64 and rounded once to float32, then the group's
// scale and the codes by the activation law of the int4 GEMM (`svdq_int4_quantize`'s).
template <int kIn>
__global__ __launch_bounds__(kEncThreads) void encode_svdq_int4_kernel(
    const void* __restrict__ w, const float* __restrict__ p, const uint16_t* __restrict__ down,
    const uint16_t* __restrict__ up, int rank, uint8_t* __restrict__ codes,
    uint16_t* __restrict__ scales, int64_t chunks, int K) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kEncThreads + threadIdx.x;
    const bool live = e < chunks;
    const int per_row = K / 8;
    const int64_t row = live ? e / per_row : 0;
    const int c = live ? static_cast<int>(e % per_row) : 0;
    float wv[8];
    load8in<kIn>(w, row * K + 8 * c, wv);
    double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int r = 0; r < rank; ++r) {
        const double u = static_cast<double>(float_of(static_cast<uint32_t>(up[row * rank + r]) << 16));
        const uint4 d = *reinterpret_cast<const uint4*>(down + static_cast<int64_t>(r) * K + 8 * c);
        const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[2 * i] = __fma_rn(u, static_cast<double>(float_of(dw[i] << 16)), acc[2 * i]);
            acc[2 * i + 1] = __fma_rn(u, static_cast<double>(float_of(dw[i] & 0xffff0000u)), acc[2 * i + 1]);
        }
    }
    float v[8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const double res = static_cast<double>(wv[i]) - acc[i];
        v[i] = static_cast<float>(res / static_cast<double>(p[8 * c + i]));
        amax = fmaxf(amax, fabsf(v[i]));
    }
    // The group's eight chunks are eight consecutive lanes (8 | 64 and groups start at 8-lane
    // boundaries since K/8 is a multiple of 8).
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const _Float16 s16 = static_cast<_Float16>(__fdiv_rn(amax, 7.0f));
    const float s = static_cast<float>(s16);
    uint32_t packed = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float q = 0.0f;
        if (s != 0.0f) q = fminf(fmaxf(__builtin_rintf(__fdiv_rn(v[i], s)), -8.0f), 7.0f);
        packed |= (static_cast<uint32_t>(static_cast<int>(q)) & 0xfu) << (4 * i);
    }
    if (!live) return;
    *reinterpret_cast<uint32_t*>(codes + row * (K / 2) + 4 * c) = packed;
    if ((c & 7) == 0) scales[row * (K / 64) + c / 8] = __builtin_bit_cast(uint16_t, s16);
}

// ------------------------------------------------------------------------------ measure

// Σ (w − d)², Σ w² (float64) and max |w − d| of a matrix `w` against its decoded float32 `d`,
// one partial a workgroup, then one workgroup folds the partials into `out` [sse, energy, max].
template <int kIn>
__global__ __launch_bounds__(kEncThreads) void measure_kernel(const void* __restrict__ w, const float* __restrict__ d,
                                                              int64_t total, double* __restrict__ partial) {
    __shared__ double red[3][kEncThreads];
    double sse = 0.0, energy = 0.0, worst = 0.0;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kEncThreads + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * kEncThreads) {
        const double x = load1in<kIn>(w, e), y = d[e];
        sse += (x - y) * (x - y);
        energy += x * x;
        worst = fmax(worst, fabs(x - y));
    }
    red[0][threadIdx.x] = sse;
    red[1][threadIdx.x] = energy;
    red[2][threadIdx.x] = worst;
    __syncthreads();
    for (int o = kEncThreads / 2; o > 0; o >>= 1) {
        if (static_cast<int>(threadIdx.x) < o) {
            red[0][threadIdx.x] += red[0][threadIdx.x + o];
            red[1][threadIdx.x] += red[1][threadIdx.x + o];
            red[2][threadIdx.x] = fmax(red[2][threadIdx.x], red[2][threadIdx.x + o]);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        partial[3 * blockIdx.x] = red[0][0];
        partial[3 * blockIdx.x + 1] = red[1][0];
        partial[3 * blockIdx.x + 2] = red[2][0];
    }
}

__global__ __launch_bounds__(64) void measure_fold_kernel(const double* __restrict__ partial, int parts,
                                                          double* __restrict__ out) {
    if (threadIdx.x != 0) return;
    double sse = 0.0, energy = 0.0, worst = 0.0;
    for (int i = 0; i < parts; ++i) {
        sse += partial[3 * i];
        energy += partial[3 * i + 1];
        worst = fmax(worst, partial[3 * i + 2]);
    }
    out[0] = sse;
    out[1] = energy;
    out[2] = worst;
}

template <template <int> class F, typename... Args>
hipError_t by_input(int in_type, Args&&... args) {
    switch (in_type) {
        case kNumF32: return F<kNumF32>::run(args...);
        case kNumBf16: return F<kNumBf16>::run(args...);
        default: return F<kNumF16>::run(args...);
    }
}

template <int kIn>
struct RotatedRun {
    static hipError_t run(const void* w, int64_t rows, int K, int8_t* q, float* scale, uint8_t* codes,
                          uint8_t* group_scale, const float* codebook, bool w4, hipStream_t s) {
        if (w4)
            hipLaunchKernelGGL((encode_rotated_kernel<kIn, true>), dim3(static_cast<uint32_t>(rows)), dim3(kEncThreads), 0, s,
                               w, K, q, scale, codes, group_scale, codebook);
        else
            hipLaunchKernelGGL((encode_rotated_kernel<kIn, false>), dim3(static_cast<uint32_t>(rows)), dim3(kEncThreads), 0,
                               s, w, K, q, scale, codes, group_scale, codebook);
        return hipGetLastError();
    }
};

template <int kIn>
struct Fp8Run {
    static hipError_t run(const void* w, int64_t rows, int K, uint8_t* q, float* scale, hipStream_t s) {
        hipLaunchKernelGGL((encode_fp8_rowwise_kernel<kIn>), dim3(static_cast<uint32_t>(rows)), dim3(kEncThreads), 0, s, w,
                           K, q, scale);
        return hipGetLastError();
    }
};

template <int kIn>
struct MxRun {
    static hipError_t run(const void* w, int64_t rows, int K, uint8_t* q, uint8_t* scale, int tiled, hipStream_t s) {
        const int64_t blocks = (rows * K / 8 + kEncThreads - 1) / kEncThreads;
        hipLaunchKernelGGL((encode_mx_kernel<kIn>), dim3(static_cast<uint32_t>(blocks)), dim3(kEncThreads), 0, s, w, rows,
                           K, q, scale, tiled);
        return hipGetLastError();
    }
};

template <int kIn>
struct Nvfp4Run {
    static hipError_t run(const void* w, int64_t rows, int K, uint32_t* amax, uint8_t* codes, uint8_t* scale,
                          float* scale_2, unsigned long long* saturated, hipStream_t s) {
        const int64_t total = rows * K;
        const int64_t reduce = std::min<int64_t>((total / 8 + kEncThreads - 1) / kEncThreads, 2048);
        hipLaunchKernelGGL((amax_kernel<kIn>), dim3(static_cast<uint32_t>(reduce)), dim3(kEncThreads), 0, s, w, total, amax);
        const int64_t blocks = total / 16;
        hipLaunchKernelGGL((encode_nvfp4_kernel<kIn>), dim3(static_cast<uint32_t>((blocks + kEncThreads - 1) / kEncThreads)),
                           dim3(kEncThreads), 0, s, w, blocks, amax, codes, scale, scale_2, saturated);
        return hipGetLastError();
    }
};

template <int kIn>
struct MeasureRun {
    static hipError_t run(const void* w, const float* d, int64_t total, double* partial, int parts, double* out,
                          hipStream_t s) {
        hipLaunchKernelGGL((measure_kernel<kIn>), dim3(static_cast<uint32_t>(parts)), dim3(kEncThreads), 0, s, w, d, total,
                           partial);
        hipLaunchKernelGGL(measure_fold_kernel, dim3(1), dim3(64), 0, s, partial, parts, out);
        return hipGetLastError();
    }
};

}  // namespace

hipError_t encode_rotated(const void* w, int in_type, int64_t rows, int K, int8_t* q, float* scale, uint8_t* codes,
                          uint8_t* group_scale, const float* codebook, bool w4, hipStream_t s) {
    return by_input<RotatedRun>(in_type, w, rows, K, q, scale, codes, group_scale, codebook, w4, s);
}

hipError_t encode_fp8_rowwise(const void* w, int in_type, int64_t rows, int K, uint8_t* q, float* scale,
                              hipStream_t s) {
    return by_input<Fp8Run>(in_type, w, rows, K, q, scale, s);
}

hipError_t encode_mx(const void* w, int in_type, int64_t rows, int K, uint8_t* q, uint8_t* scale, int tiled,
                     hipStream_t s) {
    return by_input<MxRun>(in_type, w, rows, K, q, scale, tiled, s);
}

hipError_t encode_nvfp4(const void* w, int in_type, int64_t rows, int K, uint32_t* amax, uint8_t* codes,
                        uint8_t* scale, float* scale_2, unsigned long long* saturated, hipStream_t s) {
    return by_input<Nvfp4Run>(in_type, w, rows, K, amax, codes, scale, scale_2, saturated, s);
}

hipError_t encode_svdq_int4(const void* w, int in_type, const float* p, const void* down,
                            const void* up, int rank, int64_t rows, int K, uint8_t* codes,
                            uint16_t* scales, hipStream_t s) {
    const int64_t chunks = rows * (K / 8);
    if (chunks == 0) return hipSuccess;
    const unsigned blocks = static_cast<unsigned>((chunks + kEncThreads - 1) / kEncThreads);
    const auto* d = static_cast<const uint16_t*>(down);
    const auto* u = static_cast<const uint16_t*>(up);
    if (in_type == kNumF32)
        encode_svdq_int4_kernel<kNumF32><<<blocks, kEncThreads, 0, s>>>(w, p, d, u, rank, codes, scales, chunks, K);
    else if (in_type == kNumBf16)
        encode_svdq_int4_kernel<kNumBf16><<<blocks, kEncThreads, 0, s>>>(w, p, d, u, rank, codes, scales, chunks, K);
    else
        encode_svdq_int4_kernel<kNumF16><<<blocks, kEncThreads, 0, s>>>(w, p, d, u, rank, codes, scales, chunks, K);
    return hipGetLastError();
}

hipError_t measure(const void* w, int in_type, const float* d, int64_t total, double* partial, int parts,
                   double* out, hipStream_t s) {
    return by_input<MeasureRun>(in_type, w, d, total, partial, parts, out, s);
}

}  // namespace cozyq
