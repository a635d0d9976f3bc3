// The fp8 rowwise linear for 1..4 rows in one launch (decode): the activation rows are quantized
// (internal/fp8_linear.py:56-63's law, bit for bit) inside the GEMV, so a decode step is one
// launch bound by streaming the e4m3 weight from HBM once. More rows answer NOT_SUPPORTED and the
// caller quantizes once and runs the narrow GEMM (gemm_narrow.hip).
#include "common.h"
#include "kernels.h"
#include "rotate.h"
#include "rows.h"

namespace cozyq {
namespace {

// Two choices make it run at HBM speed.
//
// The activation is loaded FIRST, into registers: a wave's loads complete in issue order, so
// activation loads issued after the weight stream would make the amax and the quantization wait
// for the whole stream. Here its arithmetic (amax, scale, codes into LDS) runs while the weights
// arrive.
//
// The weight is streamed contiguously: each load instruction reads 1 KB of one weight row (lane
// l at byte 16·l), as a plain copy does, instead of 64-byte pieces of 16 rows. The MFMA then
// multiplies 16 chunks of ONE row (A) by the same 16 chunks of the activation (B), lanes paired
// byte for byte, so D[a][b] = Σ W[chunk a]·x[chunk b] and the row's dot product is the trace of
// D (accumulated over the row's 2 KB spans). The matrix core does 16x the needed work, which at
// one row costs ~0.4 us against a ~7 us weight stream.
//
// A wave owns kRowsPerWave consecutive weight rows (one contiguous range); a thread holds 8
// consecutive activation elements of each of kChunks (kDThreads·8)-element chunks of each row.
constexpr int kXLoads = 8;
constexpr int kRowsPerWave = 2;
constexpr int kDWaves = 4;                  // waves a decode workgroup
constexpr int kDThreads = 64 * kDWaves;
constexpr int kSpanBatch = 2;  // 2 KB spans of each row a wave has in flight
// Cache policy of the weight stream (sc0 nt): each weight byte is read once per call, so its lines
// are not kept; measured 0.7 us faster than the default policy on the M = 1 decode shape.
constexpr int kStreamPolicy = 3;

template <bool kXHalf, bool kOutHalf, bool kBias, int kM, int kChunks>
__global__ __launch_bounds__(kDThreads) void fp8_decode_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ W, const float* __restrict__ ws,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int N, int K) {
    static_assert(kM * kChunks <= kXLoads, "activation registers");
    extern __shared__ __attribute__((aligned(16))) uint8_t xq[];  // kM rows of `stride` bytes
    __shared__ float red[kDWaves][kM];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int spans = (K + 2047) / 2048;
    const int stride = spans * 2048;
    const int nw = blockIdx.x * (kDWaves * kRowsPerWave) + wave * kRowsPerWave;  // the wave's first row

    // Every load is a buffer load with no branch around it (bytes past a row read as zeros): a
    // guarded load becomes a branch, and across branches the wait before the activation's first
    // use would wait for the whole weight stream.
    // 1. The activation: this thread's 8-element runs of every row.
    uint4 xv[kM][kChunks];
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(x + static_cast<int64_t>(m) * K), 0, 2 * K, 0x00020000);
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
            const int e = c * (kDThreads * 8) + tid * 8;
            xv[m][c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, 2 * e, 0, 0));
        }
    }
    asm volatile("" ::: "memory");  // the weight loads stay behind the activation's

    // 2. The weight stream: kSpanBatch 2 KB spans of each of the wave's rows, two 1 KB loads each.
    __amdgpu_buffer_rsrc_t wr[kRowsPerWave];
#pragma unroll
    for (int i = 0; i < kRowsPerWave; ++i)
        wr[i] = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(W + static_cast<int64_t>(min(nw + i, N - 1)) * K), 0, K, 0x00020000);
    uint4 wv[kRowsPerWave][kSpanBatch][2];
    auto issue = [&](int first) {
#pragma unroll
        for (int i = 0; i < kRowsPerWave; ++i)
#pragma unroll
            for (int b = 0; b < kSpanBatch; ++b)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int k = (first + b) * 2048 + h * 1024 + 16 * lane;  // >= K reads zeros
                    wv[i][b][h] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr[i], k, 0, kStreamPolicy));
                }
    };
    issue(0);

    // 3. Row amax (internal/fp8_linear.py:60), then codes into LDS, from the registers.
    float amax[kM];
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        amax[m] = 0.0f;
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
            const uint32_t w4[4] = {xv[m][c].x, xv[m][c].y, xv[m][c].z, xv[m][c].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                amax[m] = fmaxf(amax[m], fabsf(widen<kXHalf>(w4[i] & 0xffffu)));
                amax[m] = fmaxf(amax[m], fabsf(widen<kXHalf>(w4[i] >> 16)));
            }
        }
        amax[m] = wave_max(amax[m]);
        if (lane == 0) red[wave][m] = amax[m];
    }
    __syncthreads();
    // Every thread reduces the waves' maxima itself (no second barrier); thread m keeps row m's
    // scale for the epilogue.
    float scale[kM];
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        float v = red[0][m];
#pragma unroll
        for (int w = 1; w < kDWaves; ++w) v = fmaxf(v, red[w][m]);
        scale[m] = fmaxf(v / kE4m3Max, kScaleFloor);
    }
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        const float s = scale[m];
        const float rs = 1.0f / s;  // one correctly rounded reciprocal a row; div_rn per element
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
            const int e = c * (kDThreads * 8) + tid * 8;
            if (e >= stride) continue;
            const uint32_t w4[4] = {xv[m][c].x, xv[m][c].y, xv[m][c].z, xv[m][c].w};
            // The law clamps to ±448 before the cast; here |x| <= amax = 448·s, so |x / s| <=
            // 448·(1 + 2^-23) and the cast alone rounds it to 448 exactly as the clamp would.
            float q[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t h = (i & 1) ? (w4[i / 2] >> 16) : (w4[i / 2] & 0xffffu);
                q[i] = div_rn(widen<kXHalf>(h), s, rs);
            }
            *reinterpret_cast<uint2*>(xq + m * stride + e) =
                make_uint2(e4m3x4(q[0], q[1], q[2], q[3]), e4m3x4(q[4], q[5], q[6], q[7]));
        }
    }
    __syncthreads();

    // 4. Products: per row, per activation row, the trace accumulates over the spans.
    f32x4 acc[kRowsPerWave][kM];
#pragma unroll
    for (int i = 0; i < kRowsPerWave; ++i)
#pragma unroll
        for (int m = 0; m < kM; ++m) acc[i][m] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int first = 0; first < spans; first += kSpanBatch) {
        if (first != 0) issue(first);
#pragma unroll
        for (int b = 0; b < kSpanBatch; ++b) {
            if (first + b >= spans) break;
            i32x8 xb[kM];
#pragma unroll
            for (int m = 0; m < kM; ++m) {
                const uint8_t* p = xq + m * stride + (first + b) * 2048 + 16 * lane;
                const uint4 lo = *reinterpret_cast<const uint4*>(p);
                const uint4 hi = *reinterpret_cast<const uint4*>(p + 1024);
                xb[m] = i32x8{static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z),
                              static_cast<int>(lo.w), static_cast<int>(hi.x), static_cast<int>(hi.y),
                              static_cast<int>(hi.z), static_cast<int>(hi.w)};
            }
#pragma unroll
            for (int i = 0; i < kRowsPerWave; ++i) {
                const uint4 lo = wv[i][b][0], hi = wv[i][b][1];
                const i32x8 a = {static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z),
                                 static_cast<int>(lo.w), static_cast<int>(hi.x), static_cast<int>(hi.y),
                                 static_cast<int>(hi.z), static_cast<int>(hi.w)};
#pragma unroll
                for (int m = 0; m < kM; ++m) acc[i][m] = mfma_f8(a, xb[m], acc[i][m]);
            }
        }
    }

    // 5. The trace: D[a][a] sits in lane a + 16·(a/4), register a % 4; sum those 16 lanes.
    const int a = lane & 15;
    const bool diagonal = (lane >> 4) == (a >> 2);
    float dot[kRowsPerWave][kM];
#pragma unroll
    for (int i = 0; i < kRowsPerWave; ++i)
#pragma unroll
        for (int m = 0; m < kM; ++m) {
            const f32x4 d = acc[i][m];
            const int r = a & 3;
            float v = r == 0 ? d[0] : (r == 1 ? d[1] : (r == 2 ? d[2] : d[3]));
            v = diagonal ? v : 0.0f;
            v = diagonal_sum(v);
            dot[i][m] = v;
        }
    static_assert(8 % kRowsPerWave == 0, "N % 8 == 0 keeps a wave's rows whole");
    if (lane != 0 || nw >= N) return;  // N % 8 == 0: a wave's rows are all in or all out
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        const float s = scale[m];
        uint32_t o[(kRowsPerWave + 1) / 2];
#pragma unroll
        for (int i = 0; i < kRowsPerWave; ++i) {
            float v = __fmul_rn(__fmul_rn(dot[i][m], s), ws[nw + i]);
            if constexpr (kBias) v = __fadd_rn(v, widen<kOutHalf>(bias[nw + i]));
            const uint32_t h = narrow<kOutHalf>(v);
            o[i / 2] = (i & 1) ? (o[i / 2] | (h << 16)) : h;
        }
        uint16_t* dst = out + static_cast<int64_t>(m) * N + nw;
        if constexpr (kRowsPerWave == 1) {
            *dst = static_cast<uint16_t>(o[0]);
        } else if constexpr (kRowsPerWave == 2) {
            *reinterpret_cast<uint32_t*>(dst) = o[0];
        } else if constexpr (kRowsPerWave == 4) {
            *reinterpret_cast<uint2*>(dst) = make_uint2(o[0], o[1]);
        } else {
            *reinterpret_cast<uint4*>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}

// The int8 linear for 1..4 rows in one launch (reference: rotate.cu:351-407 `gemv_kernel`):
// each workgroup rotates (H256/16) and quantizes the activation rows into LDS bit for bit as the
// CPU law does (internal/int8_linear.py:422-428; the rotation's phases are rotate.h's) while its
// weight rows stream in, then takes the exact int32 dot products on the int8 MFMA and applies
// the law's epilogue ((acc·xs)·ws, one cast, + bias in the output dtype). Same structure as the
// fp8 decode above: activation loads first, the weight stream in 1 KB contiguous loads, and the
// dot product as the trace of a 16x16x64 MFMA over 16 64-byte pieces of one 1 KB span.
constexpr int kISpanBatch = 4;  // 1 KB spans of each row a wave has in flight
// Weight rows a wave owns: 4 measured 5% faster than 2 at M=1, K=3072, N=12288 on MI355X (the
// workgroup's rotation is shared by twice the rows), 8 slower.
constexpr int kIRows = 4;
// Activation registers a thread may hold (8 bf16 a uint4, 2048 elements a row a uint4 across the
// workgroup): 24, so that with the rotated values (M·K/256 floats) the widest admitted rows still
// fit one wave's 512 registers: M = 1 to K = 32768, M = 2 to 16384, M = 3 and 4 to 12288.
constexpr int kIXLoads = 24;

template <bool kXHalf, bool kOutHalf, bool kBias, int kM, int kChunks>
__global__ __launch_bounds__(kDThreads) void int8_decode_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ W, const float* __restrict__ ws,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int N, int K) {
    static_assert(kM * kChunks <= kIXLoads, "activation registers");
    using L = Layout<256>;
    constexpr int kChunks4 = (kChunks + 1) / 2;  // 4096-element rotation chunks of a row
    // The rotation's workspace; once every row is rotated, the rows' codes (`stride` bytes each,
    // zero past K) in the same bytes.
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    float* work = reinterpret_cast<float*>(smem);
    int8_t* xq = reinterpret_cast<int8_t*>(smem);
    __shared__ float red[kDWaves][kM];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int spans = (K + 1023) / 1024;
    const int stride = spans * 1024;
    const int nw = blockIdx.x * (kDWaves * kIRows) + wave * kIRows;  // the wave's first row

    // 1. The activation: this thread's 8-element runs of every row (branch-free buffer loads,
    // zeros past K), issued before the weight stream so the rotation does not wait for it.
    uint4 xv[kM][kChunks];
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(x + static_cast<int64_t>(m) * K), 0, 2 * K, 0x00020000);
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
            const int e = c * (kDThreads * 8) + tid * 8;
            xv[m][c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, 2 * e, 0, 0));
        }
    }
    asm volatile("" ::: "memory");  // the weight loads stay behind the activation's

    // 2. The weight stream: kISpanBatch 1 KB spans of each of the wave's rows.
    __amdgpu_buffer_rsrc_t wr[kIRows];
#pragma unroll
    for (int i = 0; i < kIRows; ++i)
        wr[i] = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int8_t*>(W + static_cast<int64_t>(min(nw + i, N - 1)) * K), 0, K, 0x00020000);
    // Two batches of spans alternate: the next batch's loads are issued before the current one
    // is consumed, so rows longer than a batch keep the stream busy instead of waiting out a
    // load latency per batch (M = 1, K = 32768: 52.8 -> 45.4 us; M = 4, K = 12288: 35.1 -> 29.0).
    // Rows of one batch (K <= 4096) keep the single buffer and its lower register count.
    constexpr bool kTwo = kChunks > 2;
    uint4 wa[kIRows][kISpanBatch], wb[kTwo ? kIRows : 1][kISpanBatch];
    auto issue = [&](auto& wv, int first) {
#pragma unroll
        for (int i = 0; i < kIRows; ++i)
#pragma unroll
            for (int b = 0; b < kISpanBatch; ++b) {
                const int k = (first + b) * 1024 + 16 * lane;  // >= K reads zeros
                wv[i][b] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr[i], k, 0, kStreamPolicy));
            }
    };
    issue(wa, 0);

    // 3. Each row rotated chunk by chunk through the workspace (phase 1 from the registers:
    // the thread's runs at tid·8 and 2048 + tid·8 of the chunk), its amax, then the codes.
    float rot[kM][kChunks4][16];
    float amax[kM];
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        amax[m] = 0.0f;
#pragma unroll
        for (int c4 = 0; c4 < kChunks4; ++c4) {
            const int base = c4 * kChunk;
            if (base >= K) break;
            const int width = min(kChunk, K - base);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int c = 2 * c4 + h;
                const int e = h * (kDThreads * 8) + tid * 8;  // within the chunk
                if (c >= kChunks || e >= width) continue;
                const uint32_t w4[4] = {xv[m][c].x, xv[m][c].y, xv[m][c].z, xv[m][c].w};
                float v[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[2 * i] = widen<kXHalf>(static_cast<uint16_t>(w4[i] & 0xffffu));
                    v[2 * i + 1] = widen<kXHalf>(static_cast<uint16_t>(w4[i] >> 16));
                }
                const int g = e / 256, within = e % 256;
                float* dst = work + L::at(g, within / 16, within % 16);
                *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
                *reinterpret_cast<float4*>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
            }
            rotate_lds_chunk<256, kDThreads>(work, width, tid, rot[m][c4], amax[m]);
            __syncthreads();
        }
        amax[m] = wave_max(amax[m]);
        if (lane == 0) red[wave][m] = amax[m];
    }
    __syncthreads();
    float scale[kM];
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        float v = red[0][m];
#pragma unroll
        for (int w = 1; w < kDWaves; ++w) v = fmaxf(v, red[w][m]);
        scale[m] = fmaxf(v / 127.0f, kScaleFloor);
    }
    // The codes: the thread's 16-run (group tid / 16, run tid % 16) of each chunk; zeros past K.
    const int g = tid / 16, hi = tid % 16;
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        const float s = scale[m];
        const float rs = 1.0f / s;
        const bool fast = s < __builtin_huge_valf();  // an infinite scale divides
#pragma unroll
        for (int c4 = 0; c4 < kChunks4; ++c4) {
            const int at = c4 * kChunk + g * 256 + hi * 16;
            if (at >= stride) continue;
            uint32_t packed[4] = {0, 0, 0, 0};
            if (at < K) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int8_t c = fast ? q8<true>(rot[m][c4][i], s, rs) : q8<false>(rot[m][c4][i], s, rs);
                    packed[i / 4] |= static_cast<uint32_t>(static_cast<uint8_t>(c)) << (8 * (i % 4));
                }
            }
            *reinterpret_cast<uint4*>(xq + m * stride + at) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
        }
    }
    __syncthreads();

    // 4. Products: per weight row, per activation row, the trace accumulates over the spans.
    i32x4 acc[kIRows][kM];
#pragma unroll
    for (int i = 0; i < kIRows; ++i)
#pragma unroll
        for (int m = 0; m < kM; ++m) acc[i][m] = i32x4{0, 0, 0, 0};
    auto consume = [&](const auto& wv, int first) {
#pragma unroll
        for (int b = 0; b < kISpanBatch; ++b) {
            if (first + b >= spans) break;
            i32x4 xb[kM];
#pragma unroll
            for (int m = 0; m < kM; ++m)
                xb[m] = *reinterpret_cast<const i32x4*>(xq + m * stride + (first + b) * 1024 + 16 * lane);
#pragma unroll
            for (int i = 0; i < kIRows; ++i) {
                const i32x4 a = __builtin_bit_cast(i32x4, wv[i][b]);
#pragma unroll
                for (int m = 0; m < kM; ++m) acc[i][m] = mfma_i8(a, xb[m], acc[i][m]);
            }
        }
    };
    if constexpr (kTwo) {
        for (int first = 0; first < spans; first += 2 * kISpanBatch) {
            if (first + kISpanBatch < spans) issue(wb, first + kISpanBatch);
            consume(wa, first);
            if (first + kISpanBatch >= spans) break;
            if (first + 2 * kISpanBatch < spans) issue(wa, first + 2 * kISpanBatch);
            consume(wb, first + kISpanBatch);
        }
    } else {
        consume(wa, 0);  // K <= 4096: one batch holds every span
    }

    // 5. The trace: D[a][a] sits in lane a + 16·(a/4), register a % 4; sum those 16 lanes.
    const int a = lane & 15;
    const bool diagonal = (lane >> 4) == (a >> 2);
    int dot[kIRows][kM];
#pragma unroll
    for (int i = 0; i < kIRows; ++i)
#pragma unroll
        for (int m = 0; m < kM; ++m) {
            const i32x4 d = acc[i][m];
            const int r = a & 3;
            int v = r == 0 ? d[0] : (r == 1 ? d[1] : (r == 2 ? d[2] : d[3]));
            v = diagonal ? v : 0;
            v = diagonal_sum(v);
            dot[i][m] = v;
        }
    if (lane != 0 || nw >= N) return;  // N % 4 == 0: a wave's rows are all in or all out
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        uint32_t o[(kIRows + 1) / 2];
#pragma unroll
        for (int i = 0; i < kIRows; ++i) {
            // internal/int8_linear.py:445-448 then :276: (acc·xs)·ws, cast, + bias in the output dtype.
            const float v = __fmul_rn(__fmul_rn(static_cast<float>(dot[i][m]), scale[m]), ws[nw + i]);
            uint32_t h = narrow<kOutHalf>(v);
            if constexpr (kBias)
                h = narrow<kOutHalf>(__fadd_rn(widen<kOutHalf>(static_cast<uint16_t>(h)), widen<kOutHalf>(bias[nw + i])));
            o[i / 2] = (i & 1) ? (o[i / 2] | (h << 16)) : h;
        }
        uint16_t* dst = out + static_cast<int64_t>(m) * N + nw;
        static_assert(kIRows == 4, "the store below writes four outputs");
        *reinterpret_cast<uint2*>(dst) = make_uint2(o[0], o[1]);
    }
}

template <bool kXHalf, bool kOutHalf, bool kBias>
hipError_t launch_int8_decode(const uint16_t* x, const int8_t* w, const float* ws,
                              const uint16_t* bias, uint16_t* out, int M, int N, int K,
                              hipStream_t s) {
    const int blocks = (N + kDWaves * kIRows - 1) / (kDWaves * kIRows);
    const int64_t codes = static_cast<int64_t>(M) * ((K + 1023) / 1024) * 1024;
    const int64_t work = static_cast<int64_t>(Layout<256>::kFloats) * 4;
    const int64_t lds = codes > work ? codes : work;
    const int chunks = (K + kDThreads * 8 - 1) / (kDThreads * 8);
#define COZYQ_ROWS(R, C)                                                                           \
    if (M == R && chunks <= C) {                                                                   \
        int8_decode_kernel<kXHalf, kOutHalf, kBias, R, C><<<blocks, kDThreads, lds, s>>>(x, w, ws, bias, out, N, K); \
        return hipGetLastError();                                                                  \
    }
    COZYQ_ROWS(1, 2)
    COZYQ_ROWS(1, 8)
    COZYQ_ROWS(1, 16)
    COZYQ_ROWS(2, 2)
    COZYQ_ROWS(2, 4)
    COZYQ_ROWS(2, 8)
    COZYQ_ROWS(3, 2)
    COZYQ_ROWS(3, 6)
    COZYQ_ROWS(4, 2)
    COZYQ_ROWS(4, 6)
#undef COZYQ_ROWS
    return hipErrorNotSupported;
}

template <bool kXHalf, bool kOutHalf, bool kBias>
hipError_t launch_decode(const uint16_t* x, const uint8_t* w, const float* ws,
                         const uint16_t* bias, uint16_t* out, int M, int N, int K, hipStream_t s) {
    const int blocks = (N + kDWaves * kRowsPerWave - 1) / (kDWaves * kRowsPerWave);
    const int64_t lds = static_cast<int64_t>(M) * ((K + 2047) / 2048) * 2048;
    const int chunks = (K + kDThreads * 8 - 1) / (kDThreads * 8);
#define COZYQ_ROWS(R, C)                                                                           \
    if (M == R && chunks <= C) {                                                                   \
        fp8_decode_kernel<kXHalf, kOutHalf, kBias, R, C><<<blocks, kDThreads, lds, s>>>(x, w, ws, bias, out, N, K); \
        return hipGetLastError();                                                                  \
    }
    COZYQ_ROWS(1, 2)
    COZYQ_ROWS(1, 8)
    COZYQ_ROWS(2, 2)
    COZYQ_ROWS(2, 4)
    COZYQ_ROWS(3, 2)
    COZYQ_ROWS(4, 2)
#undef COZYQ_ROWS
    return hipErrorNotSupported;
}

}  // namespace

hipError_t fp8_linear_small(const void* x, bool x_half, const uint8_t* w, const float* ws,
                            const void* bias, void* out, bool out_half, int M, int N, int K,
                            hipStream_t s) {
    // 1..4 rows whose activation fits the registers; the rest is quantize + narrow GEMM.
    if (M < 1 || M > 4 || static_cast<int64_t>(M) * K > kXLoads * kDThreads * 8) return hipErrorNotSupported;
    auto xp = static_cast<const uint16_t*>(x);
    auto bp = static_cast<const uint16_t*>(bias);
    auto op = static_cast<uint16_t*>(out);
#define COZYQ_CASE(XH, OH, B)                                                                      \
    if (x_half == XH && out_half == OH && (bias != nullptr) == B)                                  \
        return launch_decode<XH, OH, B>(xp, w, ws, bp, op, M, N, K, s);
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

int int8_gemv_max_k(int M) {
    static constexpr int kMaxKByRows[5] = {0, 32768, 16384, 12288, 12288};
    return M >= 1 && M <= 4 ? kMaxKByRows[M] : 0;
}

hipError_t int8_linear_small(const void* x, bool x_half, const int8_t* w, const float* ws,
                             const void* bias, void* out, bool out_half, int M, int N, int K,
                             hipStream_t s) {
    // 1..4 rows whose activation and rotated values fit the registers (int8_gemv_max_k); the rest
    // is quantize + GEMM.
    if (M < 1 || M > 4 || K > int8_gemv_max_k(M)) return hipErrorNotSupported;
    auto xp = static_cast<const uint16_t*>(x);
    auto bp = static_cast<const uint16_t*>(bias);
    auto op = static_cast<uint16_t*>(out);
#define COZYQ_CASE(XH, OH, B)                                                                      \
    if (x_half == XH && out_half == OH && (bias != nullptr) == B)                                  \
        return launch_int8_decode<XH, OH, B>(xp, w, ws, bp, op, M, N, K, s);
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
