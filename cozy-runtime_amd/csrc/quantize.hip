// Per-token activation quantization for gfx950: the block-Hadamard rotation with int8
// quantization, the rowwise E4M3 quantization and the MX (E8M0 per 32) quantization.
//
// Each kernel reproduces the reference's CPU torch law bit for bit: the rotation's float32
// additions in the law's stage order and association (internal/encoding/formats.py:667-671),
// correctly rounded float32 division (internal/int8_linear.py:427, internal/fp8_linear.py:
// 62-63), round-half-even and the casts of `common.h`. All three are HBM-bound: one read of the
// 16-bit rows, one write of the codes.
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "rotate.h"
#include "rows.h"

namespace cozyq {
namespace {

constexpr int kThreads = 256;
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);  // rows.h: DPP, every lane of the workgroup active
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) m = fmaxf(m, red[w]);
    __syncthreads();
    return m;
}

// Loads 8 consecutive 16-bit values as floats.
template <bool kHalf>
__device__ __forceinline__ void load8(const uint16_t* p, float* v) {
    const uint4 raw = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = widen<kHalf>(static_cast<uint16_t>(w[i] & 0xffffu));
        v[2 * i + 1] = widen<kHalf>(static_cast<uint16_t>(w[i] >> 16));
    }
}

__device__ __forceinline__ float block_sum(float v, float* red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) m += red[w];
    __syncthreads();
    return m;
}

// A float32 value rounded to the rows' dtype and widened back (an eager op's output).
template <bool kHalf>
__device__ __forceinline__ float in_dtype(float v) {
    return widen<kHalf>(narrow<kHalf>(v));
}

// The producer's prologue (`Prologue`, kernels.h; reference rotate.cu:195-282) is computed in
// float32 before the rotation, in the reference kernel's order of operations.
constexpr int kNormLayer = 1;
constexpr int kActGelu = 1, kActGeluTanh = 2, kActSitu = 3, kActSwiglu = 4;

__device__ __forceinline__ bool halves(const Prologue& p) {
    return p.act == kActSitu || (p.act == kActSwiglu && p.up == nullptr);
}

// Elements e..e+7 of row `row` after the prologue; `mean` and `rstd` are the row's norm
// statistics (mean 0 for the RMS norm).
template <bool kHalf>
__device__ __forceinline__ void load8_prologue(const Prologue& p, const uint16_t* x, int row,
                                               int K, int e, float mean, float rstd, float* v) {
    if (halves(p)) {
        const uint16_t* xr = x + static_cast<int64_t>(row) * (2 * K);
        float h[8], g[8];
        load8<kHalf>(xr + e, h);
        load8<kHalf>(xr + K + e, g);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (p.act == kActSitu) {
                // rotate.cu:252: (4 tanh(g/4) / (1 + e^-g)) · (25 tanh(h/25))
                v[i] = (4.0f * tanhf(g[i] * 0.25f) / (1.0f + expf(-g[i]))) * (25.0f * tanhf(h[i] / 25.0f));
            } else {
                // rotate.cu:271-282: silu(gate) in the row dtype (IEEE divide), times up, rounded again
                const float silu = in_dtype<kHalf>(g[i] / (1.0f + expf(-g[i])));
                v[i] = in_dtype<kHalf>(silu * h[i]);
            }
        }
        return;
    }
    const int64_t at = static_cast<int64_t>(row) * K + e;
    load8<kHalf>(x + at, v);
    if (p.act == kActSwiglu) {  // gate rows in x, up rows in `up` (rotate.cu:260-268)
        float u[8];
        load8<kHalf>(p.up + at, u);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float silu = in_dtype<kHalf>(v[i] / (1.0f + expf(-v[i])));
            v[i] = in_dtype<kHalf>(silu * u[i]);
        }
        return;
    }
    if (p.norm != 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (v[i] - mean) * rstd;
    }
    const int64_t entry = row / p.rows_per_entry;
    if (p.scale != nullptr) {
        float m[8];
        load8<kHalf>(p.scale + entry * p.scale_stride + e, m);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] *= 1.0f + m[i];
    }
    if (p.shift != nullptr) {
        float m[8];
        load8<kHalf>(p.shift + entry * p.shift_stride + e, m);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] += m[i];
    }
    if (p.act == kActGelu) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.5f * v[i] * (1.0f + erff(v[i] * 0.70710678f));
    } else if (p.act == kActGeluTanh) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float y = v[i];
            v[i] = 0.5f * y * (1.0f + tanhf(0.79788456f * (y + 0.044715f * y * y * y)));
        }
    }
}

// The row's norm statistics (rotate.cu:204-221): the mean (layer norm; 0 for RMS) and
// rsqrt(Σ(x - mean)² / K + eps) over x's K elements, every thread of the block taking part.
template <bool kHalf>
__device__ __forceinline__ float2 norm_stats(const Prologue& p, const uint16_t* x, int row, int K,
                                             float* red) {
    if (p.norm == 0) return make_float2(0.0f, 1.0f);
    const uint16_t* xr = x + static_cast<int64_t>(row) * K;
    float mean = 0.0f;
    if (p.norm == kNormLayer) {
        float sum = 0.0f;
        for (int e = threadIdx.x * 8; e < K; e += blockDim.x * 8) {
            float v[8];
            load8<kHalf>(xr + e, v);
#pragma unroll
            for (int i = 0; i < 8; ++i) sum += v[i];
        }
        mean = block_sum(sum, red) / static_cast<float>(K);
    }
    float squares = 0.0f;
    for (int e = threadIdx.x * 8; e < K; e += blockDim.x * 8) {
        float v[8];
        load8<kHalf>(xr + e, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float d = v[i] - mean;
            squares += d * d;
        }
    }
    const float total = block_sum(squares, red);
    return make_float2(mean, rsqrtf(total / static_cast<float>(K) + p.eps));
}


// Rotation by H_kRot (256: H4^⊗4 then ·1/16; 128: H2⊗H4^⊗3 unnormalized) and per-row int8.
// One block per row; kMaxChunks bounds the row's 4096-element chunks held in registers.
template <bool kHalf, int kRot, int kMaxChunks, bool kPro = false>
__global__ __launch_bounds__(kThreads) void rotate_quantize_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ scales, int K,
    Prologue pro) {
    using L = Layout<kRot>;
    __shared__ __attribute__((aligned(16))) float lds[L::kFloats];
    __shared__ float red[kThreads / 64];
    const int row = blockIdx.x, tid = threadIdx.x;
    const uint16_t* xr = x + static_cast<int64_t>(row) * K;
    float2 stats = make_float2(0.0f, 1.0f);
    if constexpr (kPro) stats = norm_stats<kHalf>(pro, x, row, K, red);
    const int chunks = (K + kChunk - 1) / kChunk;
    float out[kMaxChunks][16];
    float amax = 0.0f;
    // Without a prologue the whole row is loaded first (branch-free buffer loads, zeros past K):
    // loaded chunk by chunk, each chunk waited out its own load latency behind the previous
    // chunk's rotation (quantize + few-row GEMV, graph replays: M=1 K=32768 46.9 -> 45.1 us,
    // M=4 K=12288 16.6 -> 16.5; one chunk, K <= 4096, unchanged).
    constexpr int kRuns = kChunk / (kThreads * 8);  // a thread's 8-element runs of a chunk
    uint4 xv[kPro ? 1 : kMaxChunks][kRuns];
    if constexpr (!kPro) {
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(xr), 0, 2 * K, 0x00020000);
#pragma unroll
        for (int c = 0; c < kMaxChunks; ++c)
#pragma unroll
            for (int h = 0; h < kRuns; ++h)
                xv[c][h] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                    xrs, 2 * (c * kChunk + h * kThreads * 8 + tid * 8), 0, 0));
    }

#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
        if (c >= chunks) break;
        const int base = c * kChunk;
        const int width = min(kChunk, K - base);
        // Phase 1: the chunk into LDS, 16 bytes a load.
#pragma unroll
        for (int h = 0; h < kRuns; ++h) {
            const int e = h * kThreads * 8 + tid * 8;
            if (e >= width) break;
            float v[8];
            if constexpr (kPro) {
                load8_prologue<kHalf>(pro, x, row, K, base + e, stats.x, stats.y, v);
            } else {
                const uint32_t w[4] = {xv[c][h].x, xv[c][h].y, xv[c][h].z, xv[c][h].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[2 * i] = widen<kHalf>(static_cast<uint16_t>(w[i] & 0xffffu));
                    v[2 * i + 1] = widen<kHalf>(static_cast<uint16_t>(w[i] >> 16));
                }
            }
            const int g = e / kRot, within = e % kRot;
            float* dst = lds + L::at(g, within / 16, within % 16);
            *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            *reinterpret_cast<float4*>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
        }
        rotate_lds_chunk<kRot, kThreads>(lds, width, tid, out[c], amax);
        __syncthreads();
    }
    amax = block_max(amax, red);
    const float scale = fmaxf(amax / 127.0f, kScaleFloor);
    if (tid == 0) scales[row] = kRot == 128 ? scale * 0.08838834764831845f : scale;
    int8_t* qr = q + static_cast<int64_t>(row) * K;
    const float rs = 1.0f / scale;
    auto emit = [&](auto fast) {
#pragma unroll
        for (int c = 0; c < kMaxChunks; ++c) {
            if (c >= chunks) break;
            const int base = c * kChunk;
            const int groups = min(kChunk, K - base) / kRot;
            const int g = tid / L::kRuns, hi = tid % L::kRuns;
            if (g >= groups) continue;
            uint32_t packed[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t word = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    word |= static_cast<uint32_t>(static_cast<uint8_t>(
                                q8<decltype(fast)::value>(out[c][4 * i + j], scale, rs))) << (8 * j);
                packed[i] = word;
            }
            *reinterpret_cast<uint4*>(qr + base + g * kRot + hi * 16) =
                make_uint4(packed[0], packed[1], packed[2], packed[3]);
        }
    };
    if (scale < __builtin_huge_valf()) emit(std::true_type{}); else emit(std::false_type{});
}

// Rows of at most kRowMaxK elements with no prologue: one wave per row (rows.h), no workgroup
// barrier, and each wave's next row loaded while it rotates and quantizes the current one, so a
// CU keeps ~12 rows (72 KB at K = 3072) of loads in flight.
constexpr int kRowWaves = 4;

template <bool kHalf, int kRot>
__global__ __launch_bounds__(64 * kRowWaves) void row_quantize_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ scales, int M, int K) {
    __shared__ __attribute__((aligned(16))) float lds[kRowWaves][kRowLdsFloats<kRot> > 0 ? kRowLdsFloats<kRot> : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int stride = gridDim.x * kRowWaves;
    int row = blockIdx.x * kRowWaves + wave;
    if (row >= M) return;
    uint4 a[kRowLoads], b[kRowLoads];
    auto view = [&](int r) { return row_view(x + static_cast<int64_t>(min(r, M - 1)) * K, K); };
    row_loads(view(row), lane, a);
    // Two rows a trip with the buffers' roles swapped: the next row's loads (clamped to the last
    // row, so the loads stay branch-free) are issued before the current row is worked on.
    while (true) {
        row_loads(view(row + stride), lane, b);
        quantize_row_wave<kHalf, kRot>(a, K, lane, lds[wave], q + static_cast<int64_t>(row) * K, scales + row);
        row += stride;
        if (row >= M) break;
        row_loads(view(row + stride), lane, a);
        quantize_row_wave<kHalf, kRot>(b, K, lane, lds[wave], q + static_cast<int64_t>(row) * K, scales + row);
        row += stride;
        if (row >= M) break;
    }
}

// Per-row int8 without rotation (build lane): s = max(amax/127, 1e-12), q = clamp(rne(x/s)).
// Per-row E4M3 (fp8 = true): s = max(amax/448, 1e-12), q = e4m3(clamp(x/s, ±448)).
// One block per row; two passes over the row (the second from cache).
template <bool kHalf, bool kFp8, bool kPro = false>
__global__ __launch_bounds__(kThreads) void rowwise_quantize_kernel(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ q, float* __restrict__ scales, int K,
    Prologue pro) {
    __shared__ float red[kThreads / 64];
    const int row = blockIdx.x, tid = threadIdx.x;
    const uint16_t* xr = x + static_cast<int64_t>(row) * K;
    float2 stats = make_float2(0.0f, 1.0f);
    if constexpr (kPro) stats = norm_stats<kHalf>(pro, x, row, K, red);
    auto load = [&](int e, float* v) {
        if constexpr (kPro)
            load8_prologue<kHalf>(pro, x, row, K, e, stats.x, stats.y, v);
        else
            load8<kHalf>(xr + e, v);
    };
    float amax = 0.0f;
    for (int e = tid * 8; e < K; e += kThreads * 8) {
        float v[8];
        load(e, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    }
    amax = block_max(amax, red);
    const float scale = fmaxf(amax / (kFp8 ? kE4m3Max : 127.0f), kScaleFloor);
    if (tid == 0) scales[row] = scale;
    uint8_t* qr = q + static_cast<int64_t>(row) * K;
    const float rs = 1.0f / scale;
    auto emit = [&](auto fast) {
        constexpr bool kFast = decltype(fast)::value;
        for (int e = tid * 8; e < K; e += kThreads * 8) {
            float v[8];
            load(e, v);
            uint32_t word[2] = {0, 0};
            if constexpr (kFp8) {
                float r[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    r[i] = fminf(fmaxf(kFast ? div_rn(v[i], scale, rs) : v[i] / scale, -kE4m3Max), kE4m3Max);
                word[0] = e4m3x4(r[0], r[1], r[2], r[3]);
                word[1] = e4m3x4(r[4], r[5], r[6], r[7]);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    word[i / 4] |= static_cast<uint32_t>(static_cast<uint8_t>(q8<kFast>(v[i], scale, rs))) << (8 * (i % 4));
            }
            *reinterpret_cast<uint2*>(qr + e) = make_uint2(word[0], word[1]);
        }
    };
    if (scale < __builtin_huge_valf()) emit(std::true_type{}); else emit(std::false_type{});
}

// fp8 rows of at most kRowMaxK elements with no prologue: one wave per row (rows.h's loads and
// wave maximum), the same law as rowwise_quantize_kernel<fp8> element for element (s = max(amax /
// 448, floor), codes e4m3(clamp(x / s, ±448))), with no workgroup barrier and no second pass.
template <bool kHalf>
__global__ __launch_bounds__(256) void fp8_row_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
                                                      float* __restrict__ scales, int M, int K) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;  // a whole wave
    uint4 raw[kRowLoads];
    row_loads(row_view(x + static_cast<int64_t>(row) * K, K), lane, raw);
    float v[kRowLoads][8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kRowLoads; ++i) {
        unpack8<kHalf>(raw[i], v[i]);
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[i][j]));
    }
    amax = wave_max(amax);
    const float scale = fmaxf(amax / kE4m3Max, kScaleFloor);
    if (lane == 0) scales[row] = scale;
    uint8_t* qr = q + static_cast<int64_t>(row) * K;
    const float rs = 1.0f / scale;
    auto emit = [&](auto fast) {
        constexpr bool kFast = decltype(fast)::value;
#pragma unroll
        for (int i = 0; i < kRowLoads; ++i) {
            const int e = 8 * (lane + 64 * i);
            if (e >= K) continue;
            float r[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                r[j] = fminf(fmaxf(kFast ? div_rn(v[i][j], scale, rs) : v[i][j] / scale, -kE4m3Max), kE4m3Max);
            *reinterpret_cast<uint2*>(qr + e) = make_uint2(e4m3x4(r[0], r[1], r[2], r[3]), e4m3x4(r[4], r[5], r[6], r[7]));
        }
    };
    if (scale < __builtin_huge_valf()) emit(std::true_type{}); else emit(std::false_type{});
}

// MX quantization: 4 threads per 32-element block, 8 elements each.
template <bool kHalf>
__global__ __launch_bounds__(kThreads) void mx_quantize_kernel(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ q, uint8_t* __restrict__ scales,
    int64_t total8) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    // Every lane takes part in the shuffles; lanes past the end work on a clamped copy.
    const int64_t at = i < total8 ? i : total8 - 1;
    float v[8];
    load8<kHalf>(x + at * 8, v);
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(v[k]));
    amax = fmaxf(amax, dpp_move<0xB1>(amax));  // the block's 4 lanes: quad_perm 1,0,3,2
    amax = fmaxf(amax, dpp_move<0x4E>(amax));  // quad_perm 2,3,0,1
    const uint32_t byte = mx_byte(amax);
    // x / 2^(byte-127) as x · 2^(127-byte): the same real number, rounded once either way.
    const float inv = byte >= 254 ? float_of(1u << 22) : float_of((254u - byte) << 23);
    if (i >= total8) return;
    float r[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) r[k] = fminf(fmaxf(v[k] * inv, -kE4m3Max), kE4m3Max);
    *reinterpret_cast<uint2*>(q + i * 8) =
        make_uint2(e4m3x4(r[0], r[1], r[2], r[3]), e4m3x4(r[4], r[5], r[6], r[7]));
    if ((i & 3) == 0) scales[i >> 2] = static_cast<uint8_t>(byte);
}

template <bool kHalf, int kRot, bool kPro>
hipError_t launch_rotated(const void* x, int8_t* q, float* scales, int M, int K,
                          const Prologue& pro, hipStream_t s) {
    const int chunks = (K + kChunk - 1) / kChunk;
    const dim3 grid(M), block(kThreads);
    auto xp = static_cast<const uint16_t*>(x);
    if (chunks <= 1)
        rotate_quantize_kernel<kHalf, kRot, 1, kPro><<<grid, block, 0, s>>>(xp, q, scales, K, pro);
    else if (chunks <= 2)
        rotate_quantize_kernel<kHalf, kRot, 2, kPro><<<grid, block, 0, s>>>(xp, q, scales, K, pro);
    else if (chunks <= 4)
        rotate_quantize_kernel<kHalf, kRot, 4, kPro><<<grid, block, 0, s>>>(xp, q, scales, K, pro);
    else
        rotate_quantize_kernel<kHalf, kRot, 8, kPro><<<grid, block, 0, s>>>(xp, q, scales, K, pro);
    return hipGetLastError();
}

template <bool kHalf, bool kFp8>
hipError_t launch_rowwise(const void* x, uint8_t* q, float* scales, int M, int K,
                          const Prologue* pro, hipStream_t s) {
    auto xp = static_cast<const uint16_t*>(x);
    if constexpr (kFp8) {
        if (pro == nullptr && K <= kRowMaxK && K % 8 == 0) {
            fp8_row_kernel<kHalf><<<(M + 3) / 4, 256, 0, s>>>(xp, q, scales, M, K);
            return hipGetLastError();
        }
    }
    if (pro != nullptr)
        rowwise_quantize_kernel<kHalf, kFp8, true><<<M, kThreads, 0, s>>>(xp, q, scales, K, *pro);
    else
        rowwise_quantize_kernel<kHalf, kFp8, false><<<M, kThreads, 0, s>>>(xp, q, scales, K, Prologue{});
    return hipGetLastError();
}

}  // namespace

hipError_t rotate_quantize(const void* x, bool x_half, int8_t* q, float* scales, int M, int K,
                           int rotation, const Prologue* pro, hipStream_t s) {
    if (M == 0) return hipSuccess;
    if (pro != nullptr) {
        if (rotation != 256) return hipErrorInvalidValue;
        return x_half ? launch_rotated<true, 256, true>(x, q, scales, M, K, *pro, s)
                      : launch_rotated<false, 256, true>(x, q, scales, M, K, *pro, s);
    }
    const Prologue none{};
    if (K <= kRowMaxK && (rotation == 0 || rotation == 128 || rotation == 256)) {
        // 12 waves a CU: three 4-wave blocks on each of the 256 CUs, grid-strided over the rows.
        const int blocks = min((M + kRowWaves - 1) / kRowWaves, 3 * 256);
        auto xp = static_cast<const uint16_t*>(x);
#define COZYQ_ROWS(H, R) row_quantize_kernel<H, R><<<blocks, 64 * kRowWaves, 0, s>>>(xp, q, scales, M, K)
        if (rotation == 0) { if (x_half) COZYQ_ROWS(true, 0); else COZYQ_ROWS(false, 0); }
        else if (rotation == 128) { if (x_half) COZYQ_ROWS(true, 128); else COZYQ_ROWS(false, 128); }
        else { if (x_half) COZYQ_ROWS(true, 256); else COZYQ_ROWS(false, 256); }
#undef COZYQ_ROWS
        return hipGetLastError();
    }
    if (rotation == 0) {
        auto qp = reinterpret_cast<uint8_t*>(q);
        return x_half ? launch_rowwise<true, false>(x, qp, scales, M, K, nullptr, s)
                      : launch_rowwise<false, false>(x, qp, scales, M, K, nullptr, s);
    }
    if (rotation == 256)
        return x_half ? launch_rotated<true, 256, false>(x, q, scales, M, K, none, s)
                      : launch_rotated<false, 256, false>(x, q, scales, M, K, none, s);
    if (rotation == 128)
        return x_half ? launch_rotated<true, 128, false>(x, q, scales, M, K, none, s)
                      : launch_rotated<false, 128, false>(x, q, scales, M, K, none, s);
    return hipErrorInvalidValue;
}

hipError_t fp8_quantize(const void* x, bool x_half, uint8_t* q, float* scales, int M, int K,
                        const Prologue* pro, hipStream_t s) {
    if (M == 0) return hipSuccess;
    return x_half ? launch_rowwise<true, true>(x, q, scales, M, K, pro, s)
                  : launch_rowwise<false, true>(x, q, scales, M, K, pro, s);
}

hipError_t mx_quantize(const void* x, bool x_half, uint8_t* q, uint8_t* scales, int M, int K,
                       hipStream_t s) {
    const int64_t total8 = static_cast<int64_t>(M) * K / 8;
    if (total8 == 0) return hipSuccess;
    const int64_t blocks = (total8 + kThreads - 1) / kThreads;
    auto xp = static_cast<const uint16_t*>(x);
    if (x_half)
        mx_quantize_kernel<true><<<blocks, kThreads, 0, s>>>(xp, q, scales, total8);
    else
        mx_quantize_kernel<false><<<blocks, kThreads, 0, s>>>(xp, q, scales, total8);
    return hipGetLastError();
}

}  // namespace cozyq
