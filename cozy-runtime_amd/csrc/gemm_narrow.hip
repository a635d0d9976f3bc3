// The int8 and fp8 rowwise GEMMs for few rows (M <= 256) on gfx950, with the epilogues of the
// big kernels: int8 on v_mfma_i32_16x16x64_i8 (exact int32; the CPU law's (acc·xs)·ws, cast,
// then + bias in the output dtype, internal/int8_linear.py:445-448 and :276), fp8 on
// v_mfma_f32_16x16x128_f8f6f4 ((acc·xs)·ws + bias in float32, one cast). Tiles of kTM x kTN
// keep a few rows spread over ~224 workgroups: the weight stream, not the matrix core, bounds
// these shapes (at M = 256 the 58.7 MB fp8 weight is 7.3 us of HBM against 6 us of MFMA).
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

__device__ __forceinline__ float gelu_tanh(float y) {
    return 0.5f * y * (1.0f + tanhf(0.79788456f * (y + 0.044715f * y * y * y)));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_from(const uint8_t* base, int row0, int rows,
                                                          int K) {
    const int64_t span = static_cast<int64_t>(rows - row0) * K;
    const uint32_t bytes = span > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(span);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base + static_cast<int64_t>(row0) * K),
                                             0, bytes, 0x00020000);
}

template <bool kInt8, int kTM, int kTN, bool kOutHalf, bool kBias, int kEpi>
__global__ __launch_bounds__(kThreads) void narrow_kernel(
    const uint8_t* __restrict__ X, const uint8_t* __restrict__ W, const float* __restrict__ xs,
    const float* __restrict__ ws, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out,
    int64_t ldo, int M, int N, int K, int tiles_m) {
    static_assert(kTM % 32 == 0 && kTN % 32 == 0 && kTM <= 128 && kTN <= 128, "tile");
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
    const __amdgpu_buffer_rsrc_t wr = rows_from(W, n0, N, K);
    const int nk = (K + kStep - 1) / kStep;

    // Chunk tid + 256·i: row (tid + 256·i) / 8 of the tile, 16-byte column tid % 8.
    const int col = tid & 7;
    uint4 sx[kXLoads], sw[kWLoads];
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
            const uint32_t off = kb < K ? static_cast<uint32_t>(r * K + kb) : kOutOfRange;
            sw[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
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
            *reinterpret_cast<uint4*>(&lw[buf][r * kStep + swz(r, col) * 16]) = sw[i];
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

template <bool kInt8, int kTM, int kTN, bool kOutHalf, bool kBias, int kEpi>
hipError_t launch(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                  const void* bias, void* out, int64_t ldo, int M, int N, int K, hipStream_t s) {
    const int tiles_m = (M + kTM - 1) / kTM, tiles_n = (N + kTN - 1) / kTN;
    narrow_kernel<kInt8, kTM, kTN, kOutHalf, kBias, kEpi><<<tiles_m * tiles_n, kThreads, 0, s>>>(
        q, w, xs, ws, static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), ldo, M, N,
        K, tiles_m);
    return hipGetLastError();
}

template <bool kInt8, int kTM, int kTN>
hipError_t shaped(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                  const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                  int epilogue, hipStream_t s) {
    const bool b = bias != nullptr;
#define COZYQ_CASE(H, B, E) \
    if (out_half == H && b == B && epilogue == E) return launch<kInt8, kTM, kTN, H, B, E>(q, xs, w, ws, bias, out, ldo, M, N, K, s);
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

template <bool kInt8>
hipError_t narrow(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                  const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                  int epilogue, hipStream_t s) {
    if (M <= 32) return shaped<kInt8, 32, 64>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s);
    if (M <= 64) return shaped<kInt8, 64, 64>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s);
    if (M <= 128) return shaped<kInt8, 128, 64>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s);
    if (M <= 256) return shaped<kInt8, 128, 128>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s);
    return hipErrorNotSupported;
}

}  // namespace

hipError_t gemm_fp8_narrow(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                           const void* bias, void* out, int64_t ldo, bool out_half, int M, int N,
                           int K, int epilogue, hipStream_t s) {
    return narrow<false>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s);
}

hipError_t gemm_int8_narrow(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                            const void* bias, void* out, int64_t ldo, bool out_half, int M, int N,
                            int K, int epilogue, hipStream_t s) {
    return narrow<true>(reinterpret_cast<const uint8_t*>(q), xs, reinterpret_cast<const uint8_t*>(w),
                        ws, bias, out, ldo, out_half, M, N, K, epilogue, s);
}

}  // namespace cozyq
