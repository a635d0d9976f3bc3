// The fp8 rowwise linear for few rows (M <= 16) in one launch: decode-sized GEMMs are bound by
// streaming the e4m3 weight from HBM once, so this kernel issues the weight loads first, then
// quantizes the activation rows (internal/fp8_linear.py:56-63's law, bit for bit) into LDS while
// those loads are in flight, and multiplies on the fp8 MFMA with the rows as the B operand.
//
// One workgroup of 4 waves owns 16 weight rows; the waves split K in four contiguous ranges and
// their float32 partial sums are added in a fixed order through LDS. Each lane streams 32
// contiguous bytes of one weight row a K step (16 rows x 128 bytes a wave), the MFMA A layout.
#include "common.h"
#include "kernels.h"

namespace cozyq {
namespace {

constexpr int kThreads = 256;
constexpr int kBatch = 8;      // K steps of weight loads a wave keeps in flight
constexpr int kMaxBytes = 65536 + 256;  // LDS for the quantized rows: M·(K padded + 16) bytes

template <bool kXHalf, bool kOutHalf, bool kBias>
__global__ __launch_bounds__(kThreads) void fp8_small_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ W, const float* __restrict__ ws,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int M, int N, int K) {
    extern __shared__ __attribute__((aligned(16))) uint8_t xq[];  // M rows of `stride` bytes
    __shared__ float sx[16];
    __shared__ float red[kThreads / 64][16];
    __shared__ __attribute__((aligned(16))) f32x4 part[kThreads / 64][64];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int fr = lane & 15, fq = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int steps = (K + 127) / 128;
    const int stride = steps * 128 + 16;  // whole K steps plus a bank-spreading pad
    const int s0 = wave * steps / 4, s1 = (wave + 1) * steps / 4;
    const uint8_t* wrow = W + static_cast<int64_t>(min(n0 + fr, N - 1)) * K;

    // Weight loads of the first batch, ahead of everything else.
    uint4 wv[kBatch][2];
    auto issue = [&](int first) {
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int k = (first + b) * 128 + 32 * fq;
            if (first + b < s1 && k < K) {
                wv[b][0] = *reinterpret_cast<const uint4*>(wrow + k);
                wv[b][1] = k + 16 < K ? *reinterpret_cast<const uint4*>(wrow + k + 16)
                                      : make_uint4(0, 0, 0, 0);
            } else {
                wv[b][0] = make_uint4(0, 0, 0, 0);
                wv[b][1] = make_uint4(0, 0, 0, 0);
            }
        }
    };
    issue(s0);

    // Row amax: every thread strides every row; per-row block reduction.
    for (int m = 0; m < M; ++m) {
        const uint16_t* xr = x + static_cast<int64_t>(m) * K;
        float amax = 0.0f;
        for (int e = tid * 8; e < K; e += kThreads * 8) {
            const uint4 raw = *reinterpret_cast<const uint4*>(xr + e);
            const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                amax = fmaxf(amax, fabsf(widen<kXHalf>(w4[i] & 0xffffu)));
                amax = fmaxf(amax, fabsf(widen<kXHalf>(w4[i] >> 16)));
            }
        }
        for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
        if (lane == 0) red[wave][m] = amax;
    }
    __syncthreads();
    if (tid < M) {
        const float amax = fmaxf(fmaxf(red[0][tid], red[1][tid]), fmaxf(red[2][tid], red[3][tid]));
        sx[tid] = fmaxf(amax / kE4m3Max, kScaleFloor);
    }
    __syncthreads();
    // Codes into LDS; K padded to whole 128-steps with zeros.
    const int kp = steps * 128;
    for (int m = 0; m < M; ++m) {
        const uint16_t* xr = x + static_cast<int64_t>(m) * K;
        const float s = sx[m];
        for (int e = tid * 8; e < kp; e += kThreads * 8) {
            uint32_t word[2] = {0, 0};
            if (e < K) {
                const uint4 raw = *reinterpret_cast<const uint4*>(xr + e);
                const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t h = (i & 1) ? (w4[i / 2] >> 16) : (w4[i / 2] & 0xffffu);
                    const float r = fminf(fmaxf(widen<kXHalf>(h) / s, -kE4m3Max), kE4m3Max);
                    word[i / 4] |= static_cast<uint32_t>(e4m3_rn(r)) << (8 * (i % 4));
                }
            }
            *reinterpret_cast<uint2*>(xq + m * stride + e) = make_uint2(word[0], word[1]);
        }
    }
    __syncthreads();

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int first = s0; first < s1; first += kBatch) {
        if (first != s0) issue(first);
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int st = first + b;
            if (st >= s1) break;
            const i32x8 a = {static_cast<int>(wv[b][0].x), static_cast<int>(wv[b][0].y),
                             static_cast<int>(wv[b][0].z), static_cast<int>(wv[b][0].w),
                             static_cast<int>(wv[b][1].x), static_cast<int>(wv[b][1].y),
                             static_cast<int>(wv[b][1].z), static_cast<int>(wv[b][1].w)};
            i32x8 bx = {0, 0, 0, 0, 0, 0, 0, 0};
            if (fr < M) {
                const uint8_t* p = xq + fr * stride + st * 128 + 32 * fq;
                const uint4 lo = *reinterpret_cast<const uint4*>(p);
                const uint4 hi = *reinterpret_cast<const uint4*>(p + 16);
                bx = i32x8{static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z),
                           static_cast<int>(lo.w), static_cast<int>(hi.x), static_cast<int>(hi.y),
                           static_cast<int>(hi.z), static_cast<int>(hi.w)};
            }
            acc = mfma_f8(a, bx, acc);
        }
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    f32x4 sum = part[0][lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
        const f32x4 p = part[w][lane];
        sum = f32x4{sum[0] + p[0], sum[1] + p[1], sum[2] + p[2], sum[3] + p[3]};
    }
    // Lane holds out[m = fr][n0 + 4·fq + r].
    const int m = fr, n = n0 + 4 * fq;
    if (m >= M || n >= N) return;
    const float s = sx[m];
    uint16_t o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float v = __fmul_rn(__fmul_rn(sum[r], s), ws[n + r]);
        if constexpr (kBias) v = __fadd_rn(v, widen<kOutHalf>(bias[n + r]));
        o[r] = narrow<kOutHalf>(v);
    }
    *reinterpret_cast<uint2*>(out + static_cast<int64_t>(m) * N + n) =
        make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16), o[2] | (static_cast<uint32_t>(o[3]) << 16));
}

}  // namespace

hipError_t fp8_linear_small(const void* x, bool x_half, const uint8_t* w, const float* ws,
                            const void* bias, void* out, bool out_half, int M, int N, int K,
                            hipStream_t s) {
    const int64_t lds = static_cast<int64_t>(M) * (((K + 127) / 128) * 128 + 16);
    if (M < 1 || M > 16 || lds > kMaxBytes) return hipErrorNotSupported;
    const int blocks = (N + 15) / 16;
    auto xp = static_cast<const uint16_t*>(x);
    auto bp = static_cast<const uint16_t*>(bias);
    auto op = static_cast<uint16_t*>(out);
#define COZYQ_CASE(XH, OH, B)                                                                      \
    if (x_half == XH && out_half == OH && (bias != nullptr) == B) {                                \
        static const hipError_t opened = hipFuncSetAttribute(                                       \
            reinterpret_cast<const void*>(&fp8_small_kernel<XH, OH, B>),                           \
            hipFuncAttributeMaxDynamicSharedMemorySize, kMaxBytes);                                \
        if (opened != hipSuccess) return opened;                                                   \
        fp8_small_kernel<XH, OH, B><<<blocks, kThreads, lds, s>>>(xp, w, ws, bp, op, M, N, K);      \
        return hipGetLastError();                                                                  \
    }
    COZYQ_CASE(false, false, false)
    COZYQ_CASE(false, false, true)
    COZYQ_CASE(false, true, false)
    COZYQ_CASE(false, true, true)
    COZYQ_CASE(true, false, false)
    COZYQ_CASE(true, false, true)
    COZYQ_CASE(true, true, false)
    COZYQ_CASE(true, true, true)
#undef COZYQ_CASE
    return hipErrorInvalidValue;
}

}  // namespace cozyq
