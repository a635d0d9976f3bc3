// The fp8 GEMMs on gfx950 MFMA: e4m3 rowwise (v_mfma_f32_16x16x128_f8f6f4) and MXFP8
// (v_mfma_scale_f32_16x16x128_f8f6f4 with the E8M0 block scales fed to the matrix core), with
// the dequantizing epilogue fused. (The int8 GEMM is gemm_i8.hip.)
//
// One workgroup of 4 waves computes a 256x256 output tile; each wave owns a 128x128 quadrant as
// 8x8 MFMA blocks of 16x16 (256 accumulator registers a lane). K advances 128 bytes a step
// through a double-buffered LDS stage (2 x 64 KB): both operands are K-contiguous rows (X is
// [M, K], W is [N, K]), loaded 16 bytes a lane with whole 128-byte lines per row, and stored
// with a 16-byte-chunk XOR swizzle so each MFMA fragment read is bank-conflict free.
// The MFMA's A operand is the W tile and its B operand the X tile, so each lane's four results
// are four consecutive output columns of one row: an 8-byte store.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace cozyq {
namespace {

constexpr int kTile = 256;        // output rows and columns per workgroup
constexpr int kStep = 128;        // K bytes per LDS stage
constexpr int kThreads = 256;
constexpr int kOperand = kTile * kStep;  // bytes of one operand's stage

enum Kind { kInt8 = 0, kFp8 = 1, kMx = 2 };

// Physical 16-byte chunk of logical chunk `c` (0..7) in LDS row `r`: the 16 rows a fragment
// read touches at one chunk land on 16 distinct 4-bank groups.
template <int kKind>
__device__ __forceinline__ int swz(int r, int c) {
    return c ^ ((r >> 1) & 7);
}

__device__ __forceinline__ float gelu_tanh(float y) {
    return 0.5f * y * (1.0f + tanhf(0.79788456f * (y + 0.044715f * y * y * y)));
}

// kEpi: 0 plain, 1 tanh-GELU, 2 raw int32 accumulators to `acc_out` (test entry; no scales read).
template <int kKind, bool kOutHalf, bool kBias, int kEpi>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(
    const uint8_t* __restrict__ X, const uint8_t* __restrict__ W, const float* __restrict__ xs,
    const float* __restrict__ ws, const uint8_t* __restrict__ xe, const uint8_t* __restrict__ we,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int32_t* __restrict__ acc_out,
    int64_t ldo, int M, int N, int K, int tiles_n) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][kOperand];
    __shared__ __attribute__((aligned(16))) uint8_t sc[2][2][kTile * 4];  // MX: [row][block]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const int m0 = tm * kTile, n0 = tn * kTile;
    const int nk = (K + kStep - 1) / kStep;
    const int kblocks = K / 32;

    // Global -> register staging: chunk tid + 256·i is row tid/8 + 32·i, 16-byte column tid%8.
    const int col = tid & 7;
    uint4 stage[2][8];
    uint32_t sstage[2] = {0, 0};
    auto load = [&](int ks) {
        const int kb = ks * kStep + col * 16;
        const bool live = kb < K;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = (tid >> 3) + 32 * i;
            const int xr = min(m0 + r, M - 1), wr = min(n0 + r, N - 1);
            stage[0][i] = live ? *reinterpret_cast<const uint4*>(X + static_cast<int64_t>(xr) * K + kb)
                               : make_uint4(0, 0, 0, 0);
            stage[1][i] = live ? *reinterpret_cast<const uint4*>(W + static_cast<int64_t>(wr) * K + kb)
                               : make_uint4(0, 0, 0, 0);
        }
        if constexpr (kKind == kMx) {
            // Each thread: one row's four E8M0 bytes (K blocks 4ks..4ks+3) of X and of W.
            const int r = tid;
            const int xr = min(m0 + r, M - 1), wr = min(n0 + r, N - 1);
            sstage[0] = *reinterpret_cast<const uint32_t*>(xe + static_cast<int64_t>(xr) * kblocks + 4 * ks);
            sstage[1] = *reinterpret_cast<const uint32_t*>(we + static_cast<int64_t>(wr) * kblocks + 4 * ks);
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = (tid >> 3) + 32 * i;
            const int off = r * kStep + swz<kKind>(r, col) * 16;
            *reinterpret_cast<uint4*>(&lds[buf][0][off]) = stage[0][i];
            *reinterpret_cast<uint4*>(&lds[buf][1][off]) = stage[1][i];
        }
        if constexpr (kKind == kMx) {
            *reinterpret_cast<uint32_t*>(&sc[buf][0][tid * 4]) = sstage[0];
            *reinterpret_cast<uint32_t*>(&sc[buf][1][tid * 4]) = sstage[1];
        }
    };

    typedef std::conditional_t<kKind == kInt8, i32x4, f32x4> Acc;
    Acc acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = Acc{0, 0, 0, 0};

    load(0);
    store(0);
    if (nk > 1) load(1);
    __syncthreads();

    const int fr = lane & 15, fq = lane >> 4;
    for (int ks = 0; ks < nk; ++ks) {
        const int cur = ks & 1;
        const uint8_t* la = lds[cur][1];  // W tile: MFMA A
        const uint8_t* lb = lds[cur][0];  // X tile: MFMA B
        if constexpr (kKind == kInt8) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                i32x4 a[8], b[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int r = wn * 128 + i * 16 + fr;
                    a[i] = *reinterpret_cast<const i32x4*>(la + r * kStep + swz<kKind>(r, h * 4 + fq) * 16);
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int r = wm * 128 + j * 16 + fr;
                    b[j] = *reinterpret_cast<const i32x4*>(lb + r * kStep + swz<kKind>(r, h * 4 + fq) * 16);
                }
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc[i][j] = mfma_i8(a[i], b[j], acc[i][j]);
            }
        } else {
            i32x8 a[8], b[8];
            int sa[8], sb[8];
            // Lane group fq takes chunks fq and fq+4 (the f8f6f4 K layout, `common.h`), so MX
            // block fq of this step is the one its E8M0 byte scales.
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int r = wn * 128 + i * 16 + fr;
                const uint8_t* row = la + r * kStep;
                const i32x4 lo = *reinterpret_cast<const i32x4*>(row + swz<kKind>(r, fq) * 16);
                const i32x4 hi = *reinterpret_cast<const i32x4*>(row + swz<kKind>(r, fq + 4) * 16);
                a[i] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                if constexpr (kKind == kMx) sa[i] = sc[cur][1][r * 4 + fq];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int r = wm * 128 + j * 16 + fr;
                const uint8_t* row = lb + r * kStep;
                const i32x4 lo = *reinterpret_cast<const i32x4*>(row + swz<kKind>(r, fq) * 16);
                const i32x4 hi = *reinterpret_cast<const i32x4*>(row + swz<kKind>(r, fq + 4) * 16);
                b[j] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                if constexpr (kKind == kMx) sb[j] = sc[cur][0][r * 4 + fq];
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if constexpr (kKind == kMx)
                        acc[i][j] = mfma_f8_scaled(a[i], b[j], acc[i][j], sa[i], sb[j]);
                    else
                        acc[i][j] = mfma_f8(a[i], b[j], acc[i][j]);
                }
        }
        if (ks + 1 < nk) {
            store(cur ^ 1);
            if (ks + 2 < nk) load(ks + 2);
        }
        __syncthreads();
    }

    // Epilogue: lane holds out[m][n..n+3] of each block.
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int m = m0 + wm * 128 + j * 16 + fr;
        if (m >= M) continue;
        if constexpr (kEpi == 2) {
            static_assert(kKind == kInt8, "raw accumulators are the int8 GEMM's");
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int n = n0 + wn * 128 + i * 16 + 4 * fq;
                if (n < N) *reinterpret_cast<i32x4*>(acc_out + static_cast<int64_t>(m) * N + n) = acc[i][j];
            }
            continue;
        }
        const float xsm = (kKind == kMx) ? 1.0f : xs[m];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int n = n0 + wn * 128 + i * 16 + 4 * fq;
            if (n >= N) continue;
            float wsv[4] = {1.0f, 1.0f, 1.0f, 1.0f};
            uint16_t bv[4] = {0, 0, 0, 0};
#pragma unroll
            for (int r = 0; r < 4; ++r) {  // scalar loads: scale and bias may be any views
                if constexpr (kKind != kMx) wsv[r] = ws[n + r];
                if constexpr (kBias) bv[r] = bias[n + r];
            }
            uint16_t o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (kKind == kInt8) {
                    // internal/int8_linear.py:445-448 then :276: (acc·xs)·ws, cast, + bias in
                    // the output dtype: each step rounded on its own, no fused multiply-add.
                    const float v = __fmul_rn(__fmul_rn(static_cast<float>(acc[i][j][r]), xsm), wsv[r]);
                    o[r] = narrow<kOutHalf>(v);
                    if constexpr (kBias) o[r] = narrow<kOutHalf>(__fadd_rn(widen<kOutHalf>(o[r]), widen<kOutHalf>(bv[r])));
                } else {
                    float v = __fmul_rn(__fmul_rn(acc[i][j][r], xsm), wsv[r]);
                    if constexpr (kBias) v = __fadd_rn(v, widen<kOutHalf>(bv[r]));
                    o[r] = narrow<kOutHalf>(v);
                }
                if constexpr (kEpi == 1) o[r] = narrow<kOutHalf>(gelu_tanh(widen<kOutHalf>(o[r])));
            }
            const uint2 packed = make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16),
                                            o[2] | (static_cast<uint32_t>(o[3]) << 16));
            *reinterpret_cast<uint2*>(out + static_cast<int64_t>(m) * ldo + n) = packed;
        }
    }
}

template <int kKind, bool kOutHalf, bool kBias, int kEpi>
hipError_t launch(const void* q, const float* xs, const void* w, const float* ws,
                  const uint8_t* xe, const uint8_t* we, const void* bias, void* out,
                  int32_t* acc_out, int64_t ldo, int M, int N, int K, hipStream_t s) {
    const int tiles_m = (M + kTile - 1) / kTile, tiles_n = (N + kTile - 1) / kTile;
    gemm_kernel<kKind, kOutHalf, kBias, kEpi><<<tiles_m * tiles_n, kThreads, 0, s>>>(
        static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(w), xs, ws, xe, we,
        static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), acc_out, ldo, M, N, K,
        tiles_n);
    return hipGetLastError();
}

template <int kKind>
hipError_t dispatch(const void* q, const float* xs, const void* w, const float* ws,
                    const uint8_t* xe, const uint8_t* we, const void* bias, void* out,
                    int64_t ldo, bool out_half, int M, int N, int K, int epilogue, hipStream_t s) {
    const bool b = bias != nullptr;
#define COZYQ_CASE(H, B, E)                                                                     \
    if (out_half == H && b == B && epilogue == E)                                               \
        return launch<kKind, H, B, E>(q, xs, w, ws, xe, we, bias, out, nullptr, ldo, M, N, K, s);
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

}  // namespace

hipError_t gemm_fp8(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                    const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                    int epilogue, hipStream_t s) {
    if (M <= 256)  // few rows: narrow tiles keep ~224 workgroups on the weight stream
        return gemm_fp8_narrow(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s);
    return dispatch<kFp8>(q, xs, w, ws, nullptr, nullptr, bias, out, ldo, out_half, M, N, K,
                          epilogue, s);
}

hipError_t gemm_mx(const uint8_t* q, const uint8_t* qe, const uint8_t* w, const uint8_t* we,
                   const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                   hipStream_t s) {
    return dispatch<kMx>(q, nullptr, w, nullptr, qe, we, bias, out, ldo, out_half, M, N, K, 0, s);
}

}  // namespace cozyq
