// The int8 and fp8 rowwise GEMMs on narrow tiles (configs 1..4), with the epilogues of the
// 256x256 kernel: int8 on v_mfma_i32_16x16x64_i8 (exact int32; the CPU law's (acc·xs)·ws, cast,
// then + bias in the output dtype, internal/int8_linear.py:445-448 and :276), fp8 on
// v_mfma_f32_16x16x128_f8f6f4 ((acc·xs)·ws + bias in float32, one cast). They serve grids the
// 256x256 tile would leave under-filled: few rows, where tiles of kTM x kTN spread the weight
// stream over hundreds of workgroups (at M = 256 the 58.7 MB fp8 weight is 7.3 us of HBM against
// 6 us of MFMA), and any shape with fewer than 160 256x256 tiles.
//
// A workgroup of 4 waves (2 x 2) owns a kTM x kTN tile; K advances 128 bytes a step through a
// double-buffered LDS stage filled from registers. Every global read is a buffer load bounded by
// the matrix (rows past M or N and bytes past K read as zeros), so no launch shape can read
// outside the operands. MFMA A is the W tile, B the X tile: each lane's four results are four
// consecutive output columns of one row.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace cozyq {
namespace {

constexpr int kStep = 128;    // K bytes a stage
constexpr int kThreads = 256;
constexpr uint32_t kOutOfRange = 0x80000000u;  // a buffer offset past num_records reads zeros

// Physical 16-byte chunk of logical chunk c (0..7) in a 128-byte LDS row r: the 16 rows one
// fragment read touches at a chunk fall on 16 distinct 4-bank groups.
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_from(const uint8_t* base, int row0, int rows,
                                                          int K) {
    const int64_t span = static_cast<int64_t>(rows - row0) * K;
    const uint32_t bytes = span > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(span);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base + static_cast<int64_t>(row0) * K),
                                             0, bytes, 0x00020000);
}

// w4a8.convrot weights (internal/prebuilt.py:437-492): 4-bit codes [N, K/2] (even k in the low
// nibble), one E4M3 group scale per 16 codes [N, K/16], and a codebook of 16 float32 levels (or
// the uniform grid q − 8). A code's int8 level is clamp(rne(level · group scale), ±127), a NaN
// product 0 — one float32 multiply, so a 256 x 16 table T[scale byte][code] holds every level.
struct W4 {
    const uint8_t* group_scale;
    const float* codebook;  // null: the uniform grid
};

// T[b][c] for b = the calling thread's index (256 threads), as 16 bytes at table + 16·b.
__device__ __forceinline__ void w4_table_row(const float* codebook, uint32_t* table, int b) {
    const float e = e4m3_value(static_cast<uint32_t>(b));
    uint32_t words[4] = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        const float level = codebook != nullptr ? codebook[c] : static_cast<float>(c - 8);
        float r = __builtin_rintf(level * e);  // torch.round: half to even
        r = __builtin_isnan(r) ? 0.0f : fminf(fmaxf(r, -127.0f), 127.0f);
        words[c / 4] |= static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int>(r))) << (8 * (c % 4));
    }
    *reinterpret_cast<uint4*>(table + 4 * b) = make_uint4(words[0], words[1], words[2], words[3]);
}

// 16 codes (8 bytes, k order) of one group with scale byte b -> their 16 int8 levels (k order),
// by byte selects from the group's table row: codes 0..7 from its low 8 bytes, 8..15 from its
// high 8, chosen per byte by the code's bit 3.
__device__ __forceinline__ uint4 w4_unpack16(uint32_t c01, uint32_t c23, const uint32_t* table,
                                             uint32_t b) {
    const uint4 t = *reinterpret_cast<const uint4*>(table + 4 * b);
    auto four = [&](uint32_t spread) {  // four codes, one a byte
        const uint32_t sel = spread & 0x07070707u;
        const uint32_t lo = __builtin_amdgcn_perm(t.y, t.x, sel);  // levels of codes 0..7
        const uint32_t hi = __builtin_amdgcn_perm(t.w, t.z, sel);  // levels of codes 8..15
        const uint32_t m = ((spread >> 3) & 0x01010101u) * 0xffu;
        return (hi & m) | (lo & ~m);
    };
    uint32_t out[4];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const uint32_t x = d ? c23 : c01;
        const uint32_t lo = x & 0x0f0f0f0fu, hi = (x >> 4) & 0x0f0f0f0fu;
        // byte i holds k = 2i (low nibble) and 2i + 1 (high): interleave into k order.
        out[2 * d] = four(__builtin_amdgcn_perm(hi, lo, 0x05010400u));
        out[2 * d + 1] = four(__builtin_amdgcn_perm(hi, lo, 0x07030602u));
    }
    return make_uint4(out[0], out[1], out[2], out[3]);
}

// kW4: W is w4a8.convrot codes (with `w4`), unpacked to int8 levels in registers on the way
// into LDS; the rest is the int8 path (kInt8 must be true).
template <bool kInt8, int kTM, int kTN, bool kOutHalf, bool kBias, int kEpi, bool kW4 = false>
__global__ __launch_bounds__(kThreads) void narrow_kernel(
    const uint8_t* __restrict__ X, const uint8_t* __restrict__ W, const float* __restrict__ xs,
    const float* __restrict__ ws, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out,
    int64_t ldo, int M, int N, int K, int tiles_m, W4 w4) {
    static_assert(kTM % 32 == 0 && kTN % 32 == 0 && kTM <= 128 && kTN <= 128, "tile");
    static_assert(!kW4 || kInt8, "w4a8 runs the int8 path");
    constexpr int kXLoads = kTM * 8 / kThreads;   // 16-byte chunks a thread stages a step
    constexpr int kWLoads = kTN * 8 / kThreads;
    constexpr int kBI = kTN / 32, kBJ = kTM / 32;  // 16x16 blocks of a wave: n by m
    __shared__ __attribute__((aligned(16))) uint8_t lx[2][kTM * kStep];
    __shared__ __attribute__((aligned(16))) uint8_t lw[2][kTN * kStep];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // M-tiles fastest: the workgroups in flight together share their weight tiles in L2.
    const int tm = blockIdx.x % tiles_m, tn = blockIdx.x / tiles_m;
    const int m0 = __builtin_amdgcn_readfirstlane(tm * kTM);
    const int n0 = __builtin_amdgcn_readfirstlane(tn * kTN);
    const __amdgpu_buffer_rsrc_t xr = rows_from(X, m0, M, K);
    // kW4: W rows are K/2 code bytes, and the group scales K/16 bytes a row.
    const __amdgpu_buffer_rsrc_t wr = rows_from(W, n0, N, kW4 ? K / 2 : K);
    const __amdgpu_buffer_rsrc_t gr = rows_from(kW4 ? w4.group_scale : W, n0, N, kW4 ? K / 16 : K);
    const int nk = (K + kStep - 1) / kStep;
    __shared__ __attribute__((aligned(16))) uint32_t table[kW4 ? 256 * 4 : 4];
    if constexpr (kW4) {
        w4_table_row(w4.codebook, table, threadIdx.x);
        __syncthreads();
    }

    // Chunk tid + 256·i: row (tid + 256·i) / 8 of the tile, 16-byte column tid % 8.
    const int col = tid & 7;
    uint4 sx[kXLoads], sw[kWLoads];
    uint32_t sg[kWLoads];  // kW4: the chunk's group scale byte (its 16 codes in sw[i].x, .y)
    auto load = [&](int ks) {
        const int kb = ks * kStep + col * 16;
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int r = (tid >> 3) + 32 * i;
            const uint32_t off = kb < K ? static_cast<uint32_t>(r * K + kb) : kOutOfRange;
            sx[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < kWLoads; ++i) {
            const int r = (tid >> 3) + 32 * i;
            if constexpr (kW4) {
                // The chunk's 16 codes (8 bytes) and its group scale: zeros past K level to 0.
                const uint32_t off = kb < K ? static_cast<uint32_t>(r * (K / 2) + kb / 2) : kOutOfRange;
                const uint32_t goff = kb < K ? static_cast<uint32_t>(r * (K / 16) + kb / 16) : kOutOfRange;
                const auto c = __builtin_amdgcn_raw_buffer_load_b64(wr, off, 0, 0);
                sw[i] = make_uint4(c[0], c[1], 0, 0);
                sg[i] = __builtin_amdgcn_raw_buffer_load_b8(gr, goff, 0, 0);
            } else {
                const uint32_t off = kb < K ? static_cast<uint32_t>(r * K + kb) : kOutOfRange;
                sw[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int r = (tid >> 3) + 32 * i;
            *reinterpret_cast<uint4*>(&lx[buf][r * kStep + swz(r, col) * 16]) = sx[i];
        }
#pragma unroll
        for (int i = 0; i < kWLoads; ++i) {
            const int r = (tid >> 3) + 32 * i;
            uint4 v = sw[i];
            if constexpr (kW4) v = w4_unpack16(sw[i].x, sw[i].y, table, sg[i] & 0xffu);
            *reinterpret_cast<uint4*>(&lw[buf][r * kStep + swz(r, col) * 16]) = v;
        }
    };

    typedef std::conditional_t<kInt8, i32x4, f32x4> Acc;
    Acc acc[kBI][kBJ];
#pragma unroll
    for (int i = 0; i < kBI; ++i)
#pragma unroll
        for (int j = 0; j < kBJ; ++j) acc[i][j] = Acc{0, 0, 0, 0};

    load(0);
    store(0);
    if (nk > 1) load(1);
    __syncthreads();

    const int fr = lane & 15, fq = lane >> 4;
    for (int ks = 0; ks < nk; ++ks) {
        const int cur = ks & 1;
        if constexpr (kInt8) {
            // 16x16x64: lane group fq supplies 16-byte chunk fq of each 64-byte K half h.
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                i32x4 a[kBI], b[kBJ];
#pragma unroll
                for (int i = 0; i < kBI; ++i) {
                    const int r = wn * (kTN / 2) + i * 16 + fr;
                    a[i] = *reinterpret_cast<const i32x4*>(&lw[cur][r * kStep + swz(r, 4 * h + fq) * 16]);
                }
#pragma unroll
                for (int j = 0; j < kBJ; ++j) {
                    const int r = wm * (kTM / 2) + j * 16 + fr;
                    b[j] = *reinterpret_cast<const i32x4*>(&lx[cur][r * kStep + swz(r, 4 * h + fq) * 16]);
                }
#pragma unroll
                for (int i = 0; i < kBI; ++i)
#pragma unroll
                    for (int j = 0; j < kBJ; ++j) acc[i][j] = mfma_i8(a[i], b[j], acc[i][j]);
            }
        } else {
        // Lane group fq reads chunks fq and fq + 4 (the f8f6f4 K layout, `common.h`).
        i32x8 a[kBI], b[kBJ];
#pragma unroll
        for (int i = 0; i < kBI; ++i) {
            const int r = wn * (kTN / 2) + i * 16 + fr;
            const uint8_t* row = &lw[cur][r * kStep];
            const i32x4 lo = *reinterpret_cast<const i32x4*>(row + swz(r, fq) * 16);
            const i32x4 hi = *reinterpret_cast<const i32x4*>(row + swz(r, fq + 4) * 16);
            a[i] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int j = 0; j < kBJ; ++j) {
            const int r = wm * (kTM / 2) + j * 16 + fr;
            const uint8_t* row = &lx[cur][r * kStep];
            const i32x4 lo = *reinterpret_cast<const i32x4*>(row + swz(r, fq) * 16);
            const i32x4 hi = *reinterpret_cast<const i32x4*>(row + swz(r, fq + 4) * 16);
            b[j] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int i = 0; i < kBI; ++i)
#pragma unroll
            for (int j = 0; j < kBJ; ++j) acc[i][j] = mfma_f8(a[i], b[j], acc[i][j]);
        }
        if (ks + 1 < nk) {
            store(cur ^ 1);
            if (ks + 2 < nk) load(ks + 2);
        }
        __syncthreads();
    }

    // Epilogue: the lane's four consecutive columns of one row, an 8-byte store.
#pragma unroll
    for (int j = 0; j < kBJ; ++j) {
        const int m = m0 + wm * (kTM / 2) + j * 16 + fr;
        if (m >= M) continue;
        const float xsm = xs[m];
#pragma unroll
        for (int i = 0; i < kBI; ++i) {
            const int n = n0 + wn * (kTN / 2) + i * 16 + 4 * fq;
            if (n >= N) continue;  // N % 8 == 0: n..n+3 are all in
            uint16_t o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (kInt8) {
                    // Each step rounded on its own, no fused multiply-add.
                    const float v = __fmul_rn(__fmul_rn(static_cast<float>(acc[i][j][r]), xsm), ws[n + r]);
                    o[r] = narrow<kOutHalf>(v);
                    if constexpr (kBias) o[r] = narrow<kOutHalf>(__fadd_rn(widen<kOutHalf>(o[r]), widen<kOutHalf>(bias[n + r])));
                } else {
                    float v = __fmul_rn(__fmul_rn(acc[i][j][r], xsm), ws[n + r]);
                    if constexpr (kBias) v = __fadd_rn(v, widen<kOutHalf>(bias[n + r]));
                    o[r] = narrow<kOutHalf>(v);
                }
                if constexpr (kEpi == 1) o[r] = narrow<kOutHalf>(gelu_tanh(widen<kOutHalf>(o[r])));
            }
            *reinterpret_cast<uint2*>(out + static_cast<int64_t>(m) * ldo + n) =
                make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16), o[2] | (static_cast<uint32_t>(o[3]) << 16));
        }
    }
}

template <bool kInt8, int kTM, int kTN, bool kOutHalf, bool kBias, int kEpi, bool kW4>
hipError_t launch(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                  const void* bias, void* out, int64_t ldo, int M, int N, int K, W4 w4,
                  hipStream_t s) {
    const int tiles_m = (M + kTM - 1) / kTM, tiles_n = (N + kTN - 1) / kTN;
    narrow_kernel<kInt8, kTM, kTN, kOutHalf, kBias, kEpi, kW4><<<tiles_m * tiles_n, kThreads, 0, s>>>(
        q, w, xs, ws, static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), ldo, M, N,
        K, tiles_m, w4);
    return hipGetLastError();
}

template <bool kInt8, int kTM, int kTN, bool kW4 = false>
hipError_t shaped(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                  const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                  int epilogue, hipStream_t s, W4 w4 = W4{nullptr, nullptr}) {
    const bool b = bias != nullptr;
#define COZYQ_CASE(H, B, E) \
    if (out_half == H && b == B && epilogue == E) return launch<kInt8, kTM, kTN, H, B, E, kW4>(q, xs, w, ws, bias, out, ldo, M, N, K, w4, s);
    COZYQ_CASE(false, false, 0)
    COZYQ_CASE(false, true, 0)
    COZYQ_CASE(true, false, 0)
    COZYQ_CASE(true, true, 0)
    COZYQ_CASE(false, false, 1)
    COZYQ_CASE(false, true, 1)
    COZYQ_CASE(true, false, 1)
    COZYQ_CASE(true, true, 1)
#undef COZYQ_CASE
    return hipErrorInvalidValue;
}

// Tile configs 1..4 (config 0 is the 256x256 kernel of gemm.hip): 128x128, 128x64, 64x64,
// 32x64 (rows x columns). Every config computes each output with the same MFMA sequence over K
// and the same epilogue.
template <bool kInt8, bool kW4 = false>
hipError_t narrow(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                  const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                  int epilogue, int config, hipStream_t s, W4 w4 = W4{nullptr, nullptr}) {
    switch (config) {
        case 1: return shaped<kInt8, 128, 128, kW4>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s, w4);
        case 2: return shaped<kInt8, 128, 64, kW4>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s, w4);
        case 3: return shaped<kInt8, 64, 64, kW4>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s, w4);
        case 4: return shaped<kInt8, 32, 64, kW4>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s, w4);
        default: return hipErrorNotSupported;
    }
}

// The unpack law over a whole weight (internal/prebuilt.py:471-492): one thread a group of 16.
__global__ __launch_bounds__(kThreads) void w4a8_unpack_kernel(const uint8_t* __restrict__ codes,
                                                               const uint8_t* __restrict__ gs,
                                                               const float* __restrict__ codebook,
                                                               int8_t* __restrict__ out, int64_t groups,
                                                               int K) {
    __shared__ __attribute__((aligned(16))) uint32_t table[256 * 4];
    w4_table_row(codebook, table, threadIdx.x);
    __syncthreads();
    const int64_t g = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (g >= groups) return;
    const int64_t per_row = K / 16;
    const int64_t row = g / per_row, grp = g % per_row;
    const uint2 c = *reinterpret_cast<const uint2*>(codes + row * (K / 2) + grp * 8);
    const uint4 v = w4_unpack16(c.x, c.y, table, gs[row * per_row + grp]);
    *reinterpret_cast<uint4*>(out + row * K + grp * 16) = v;
}

}  // namespace

hipError_t gemm_w4a8_narrow(const int8_t* q, const float* xs, const uint8_t* codes,
                            const uint8_t* group_scale, const float* codebook, const float* ws,
                            const void* bias, void* out, bool out_half, int M, int N, int K,
                            int config, hipStream_t s) {
    return narrow<true, true>(reinterpret_cast<const uint8_t*>(q), xs, codes, ws, bias, out, N,
                              out_half, M, N, K, 0, config < 0 ? narrow_config(M, N) : config, s,
                              W4{group_scale, codebook});
}

hipError_t w4a8_unpack(const uint8_t* codes, const uint8_t* group_scale, const float* codebook,
                       int8_t* out, int N, int K, hipStream_t s) {
    const int64_t groups = static_cast<int64_t>(N) * (K / 16);
    if (groups == 0) return hipSuccess;
    w4a8_unpack_kernel<<<static_cast<unsigned>((groups + kThreads - 1) / kThreads), kThreads, 0, s>>>(
        codes, group_scale, codebook, out, groups, K);
    return hipGetLastError();
}

// The largest narrow tile whose grid reaches 440 workgroups (~1.7 a CU: the sweep's best tile
// at every shape below 160 256x256 tiles had 448-768), else the smallest.
int narrow_config(int M, int N) {
    static constexpr int kRows[] = {0, 128, 128, 64, 32}, kCols[] = {0, 128, 64, 64, 64};
    for (int c = 1; c < kGemmConfigs; ++c) {
        const int64_t groups = static_cast<int64_t>((M + kRows[c] - 1) / kRows[c]) * ((N + kCols[c] - 1) / kCols[c]);
        if (groups >= 440) return c;
    }
    return kGemmConfigs - 1;
}

hipError_t gemm_fp8_narrow(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                           const void* bias, void* out, int64_t ldo, bool out_half, int M, int N,
                           int K, int epilogue, int config, hipStream_t s) {
    return narrow<false>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, config, s);
}

hipError_t gemm_int8_narrow(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                            const void* bias, void* out, int64_t ldo, bool out_half, int M, int N,
                            int K, int epilogue, int config, hipStream_t s) {
    return narrow<true>(reinterpret_cast<const uint8_t*>(q), xs, reinterpret_cast<const uint8_t*>(w),
                        ws, bias, out, ldo, out_half, M, N, K, epilogue, config, s);
}

}  // namespace cozyq
