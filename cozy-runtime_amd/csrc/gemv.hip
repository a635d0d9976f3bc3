// The few-row linears in one launch. fp8 rowwise: the GEMV for 1..4 rows (decode) and the
// row-tile kernel for 5..16 rows (and 3..4 rows of a wide weight); the activation rows are
// quantized (internal/fp8_linear.py:56-63's law, bit for bit) inside the kernel, so a decode step
// is one launch bound by streaming the e4m3 weight from HBM once. More rows answer NOT_SUPPORTED
// and the caller quantizes once and runs the narrow GEMM (gemm_narrow.hip). int8.convrot: the
// GEMV for 1..4 rows, rotation and quantization inside it.
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
    const RowEpilogue<kRowsPerWave, kBias> epi = row_epilogue<kRowsPerWave, kBias>(ws, bias, nw, N);
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
            float v = __fmul_rn(__fmul_rn(dot[i][m], s), epi.ws[i]);
            if constexpr (kBias) v = __fadd_rn(v, widen<kOutHalf>(epi.bias[i]));
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

// The fp8 rowwise linear for 5..16 rows (and 3..4 rows of a wide weight, where it outruns the
// GEMV) in one launch. Quantizing all rows in every workgroup
// costs VALU time per CU (about 4.5 operations an element), so the grid is one workgroup per CU:
// the CUs share N in 8-row units (at most 64 rows, four 16-row tiles, a workgroup) and a
// workgroup's 8 waves split K (at most 4 steps of 128 bytes each, K <= 4096). A wave loads its K
// slice of every activation row straight into the MFMA's B layout (lane l: row l%16), the
// workgroup meets once in LDS for the rows' whole amax, and each wave quantizes its slice into
// B registers (the law bit for bit, as above). The product is the plain 16x16x128 MFMA, A = 16
// weight rows, B = the activation rows (zero past M).
//
// The weight reaches the MFMA through LDS. A register load in the A layout reads 64-byte pieces
// of 16 rows, which streams at ~4.5 TB/s on MI355X; here each load is an LDS-DMA of 2 rows x
// 512 contiguous bytes (the wave's K slice of two rows) into a per-wave slot of one 16-row tile
// (two slots a wave, 128 KB a workgroup), where a row's 16-byte chunk c sits at chunk
// c ^ (row % 16), so the A-layout reads (16 rows at one chunk) hit 16 distinct bank groups.
// Tiles 0 and 1 are loaded first. Once the workgroup has met for the amax, tile 0's A operands
// are read into registers and its slot refilled with tile 2 before the quantization, and tile 1
// likewise with tile 3 after it. Measured at M=16, K=4096, N=14336 (back-to-back launches over
// 8 weight copies): 14.0 us, against 14.6 refilling each slot after its products, 16.4 refilling
// before the amax meeting (which then waits for every wave's tile 0), and 18-19 loading all
// four tiles into registers and staging them through LDS afterwards. The waves' partial sums
// meet in LDS and are added in wave order.
constexpr int kRTiles = 4;                   // 16-row weight tiles a workgroup owns at most
constexpr int kRSpan = 32;                   // 128-byte K steps a workgroup spans (K <= 4096)
constexpr uint32_t kFar = 0x7fff0000u;       // a buffer offset past every resource here (reads 0)

template <bool kXHalf, bool kOutHalf, bool kBias, int kRWaves>
__global__ __launch_bounds__(64 * kRWaves) void fp8_rows_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ W, const float* __restrict__ ws,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int M, int N, int K,
    int units, int groups) {
    constexpr int kRSteps = kRSpan / kRWaves;     // 128-byte K steps a wave owns at most
    constexpr int kRStage = 16 * 128 * kRSteps;   // one tile's slice: 16 rows x 128·kRSteps bytes
    constexpr int kChunks = 8 * kRSteps;          // 16-byte chunks of a row's slice
    constexpr int kRowsPerLoad = 64 / kChunks;    // rows one 1 KiB LDS-DMA load fills
    constexpr int kTileLoads = 16 / kRowsPerLoad;  // loads a tile takes
    static_assert(kRWaves >= kRTiles && kRWaves * kRTiles * 64 * 16 <= kRWaves * kRStage, "partials fit a slot array");
    // The two slots are separate arrays: the compiler's wait before an LDS read then covers only
    // the LDS-DMA loads into the slot read, not the ones in flight to the other.
    __shared__ __attribute__((aligned(1024))) uint8_t slot0[kRWaves * kRStage];
    __shared__ __attribute__((aligned(1024))) uint8_t slot1[kRWaves * kRStage];
    __shared__ uint32_t red[kRWaves][16];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS-DMA bases go in M0
    const int r = lane & 15, g = lane >> 4;
    // The workgroup's rows: 8-row units [u0, u1) of N's.
    const int u0 = static_cast<int>(static_cast<int64_t>(blockIdx.x) * units / groups);
    const int u1 = static_cast<int>(static_cast<int64_t>(blockIdx.x + 1) * units / groups);
    const int row0 = 8 * u0, rows = 8 * (u1 - u0);
    // The wave's 128-byte K steps [s0, s1); bytes from kend on read as zeros. Every workgroup
    // reads the whole activation, and the 32 workgroups of an XCD (b, b + 8, ...) run together:
    // rotating which wave takes which K slice by b / 8 spreads their simultaneous activation loads
    // over 8 slices instead of one (measured 14.9 -> 13.5 us at M=16, K=4096, N=14336).
    const int steps_all = (K + 127) / 128;
    const int slice = (wave + static_cast<int>(blockIdx.x >> 3)) & (kRWaves - 1);
    const int s0 = slice * steps_all / kRWaves, s1 = (slice + 1) * steps_all / kRWaves;
    const int kend = min(K, 128 * s1);
    const int kl = 128 * s0 + 16 * g;

    // 0. The epilogue's row scales and bias (wave t finishes tile t; lane l holds weight rows
    //    16t + 4g + (0..3) of activation row l%16), fetched first so the end waits on nothing.
    const int n_out = 16 * wave + 4 * g;
    const bool emits = wave < kRTiles && n_out < rows && r < M;  // rows % 8 == 0: whole 4-row groups
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ws), 0, 4 * N, 0x00020000);
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(bias), 0, kBias ? 2 * N : 0, 0x00020000);
    float wscale[4];
    uint16_t bterm[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = row0 + n_out + i;
        wscale[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, emits ? 4 * n : kFar, 0, 0));
        if constexpr (kBias) bterm[i] = __builtin_amdgcn_raw_buffer_load_b16(br, emits ? 2 * n : kFar, 0, 0);
    }

    // 1. The activation slice, B layout: step j, part p = the 8 elements at kl + 128j + 64(p/2)
    //    + 8(p%2) of row r (rows past M lie past the resource).
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), 0, 2 * M * K, 0x00020000);
    uint4 xv[kRSteps][4];
#pragma unroll
    for (int j = 0; j < kRSteps; ++j)
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int e = kl + 128 * j + 64 * (p >> 1) + 8 * (p & 1);
            const uint32_t off = e < kend ? 2u * static_cast<uint32_t>(r * K + e) : kFar;
            xv[j][p] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        }
    fence();  // the weight loads stay behind the activation's

    // 2. Weight tiles 0 and 1 by LDS-DMA: load i of tile t fills kRowsPerLoad rows of slot t
    //    (2 at 8 waves: lane l takes row 16t + 2i + l/32 and physical chunk l % 32, which holds
    //    the row's logical chunk (l % 32) ^ (row % 16) of the wave's slice).
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(W + static_cast<int64_t>(row0) * K), 0, rows * K, 0x00020000);
    uint8_t* const slot[2] = {slot0 + wave * kRStage, slot1 + wave * kRStage};
    uint32_t src[kTileLoads];
#pragma unroll
    for (int i = 0; i < kTileLoads; ++i) {
        const int row = kRowsPerLoad * i + lane / kChunks;
        const int k = 128 * s0 + 16 * ((lane % kChunks) ^ (row & 15));
        src[i] = k < kend ? static_cast<uint32_t>(row * K + k) : kFar;
    }
    auto stage = [&](int t) {
#pragma unroll
        for (int i = 0; i < kTileLoads; ++i) {
            const uint32_t off = 16 * t + kRowsPerLoad * i + lane / kChunks < rows ? src[i] + static_cast<uint32_t>(16 * t * K) : kFar;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (LdsPtr*)(slot[t & 1] + 1024 * i), 16, off, 0, 0, kStreamPolicy);
        }
    };
    stage(0);
    stage(1);

    // 4. Row amax: bf16 and fp16 magnitudes order as their bit patterns, so the maximum is
    //    taken on the integers (two a packed op); a NaN's pattern exceeds every number's, so a
    //    row holding one gets a NaN scale and NaN outputs, as the law's row does.
    typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
    u16x2 m2 = {0, 0};
#pragma unroll
    for (int j = 0; j < kRSteps; ++j)
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t d4[4] = {xv[j][p].x, xv[j][p].y, xv[j][p].z, xv[j][p].w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, d4[i] & 0x7fff7fffu));
        }
    uint32_t top = max(static_cast<uint32_t>(m2.x), static_cast<uint32_t>(m2.y));
    top = max(top, static_cast<uint32_t>(__shfl_xor(static_cast<int>(top), 16)));
    top = max(top, static_cast<uint32_t>(__shfl_xor(static_cast<int>(top), 32)));
    if (g == 0) red[wave][r] = top;
    // A bare barrier: __syncthreads() would also wait for the weight loads in flight.
    fence();
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    fence();
#pragma unroll
    for (int w = 0; w < kRWaves; ++w) top = max(top, red[w][r]);
    // Row r's scale (internal/fp8_linear.py:60-61), lane l's row l%16.
    const float s = fmaxf(widen<kXHalf>(static_cast<uint16_t>(top)) / kE4m3Max, kScaleFloor);
    const float rs = 1.0f / s;

    // Tile 0 lands (tile 1 may still be in flight behind it): its A operands go to registers
    // (row r, logical chunks 8j + g and 8j + 4 + g) and its slot takes tile 2 before the
    // quantization, so the stream does not wait on it.
    auto read_tile = [&](int t, uint4 (&a)[kRSteps][2]) {
        const uint8_t* base = slot[t & 1] + r * (16 * kChunks);
#pragma unroll
        for (int j = 0; j < kRSteps; ++j) {
            a[j][0] = *reinterpret_cast<const uint4*>(base + 16 * ((8 * j + g) ^ r));
            a[j][1] = *reinterpret_cast<const uint4*>(base + 16 * ((8 * j + 4 + g) ^ r));
        }
    };
    auto land = [&](int t, uint4 (&a)[kRSteps][2]) {
        __builtin_amdgcn_sched_barrier(0);
        fence();
        wait_vmcnt<kTileLoads>();
        fence();
        read_tile(t, a);
        fence();
        wait_lgkmcnt0();
        fence();
        stage(t + 2);
        __builtin_amdgcn_sched_barrier(0);
    };
    uint4 early[2][kRSteps][2];
    land(0, early[0]);

    // 5. Codes: B operand of step j, bytes 0-15 = elements kl + 128j + [0, 16), bytes 16-31 =
    //    + 64 + [0, 16). x / s as div_rn without the sign fix (a zero's sign adds nothing to a
    //    sum); the cast rounds |x / s| <= 448·(1 + 2^-23) to 448 as the law's clamp would.
    i32x8 codes[kRSteps];
#pragma unroll
    for (int j = 0; j < kRSteps; ++j) {
        uint32_t c[8];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t d4[4] = {xv[j][p].x, xv[j][p].y, xv[j][p].z, xv[j][p].w};
            float q[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint16_t h = static_cast<uint16_t>((i & 1) ? (d4[i / 2] >> 16) : (d4[i / 2] & 0xffffu));
                const float v = widen<kXHalf>(h);
                const float q0 = v * rs;
                q[i] = __builtin_fmaf(__builtin_fmaf(-q0, s, v), rs, q0);
            }
            c[2 * p] = e4m3x4(q[0], q[1], q[2], q[3]);
            c[2 * p + 1] = e4m3x4(q[4], q[5], q[6], q[7]);
        }
        codes[j] = i32x8{static_cast<int>(c[0]), static_cast<int>(c[1]), static_cast<int>(c[2]),
                         static_cast<int>(c[3]), static_cast<int>(c[4]), static_cast<int>(c[5]),
                         static_cast<int>(c[6]), static_cast<int>(c[7])};
    }

    land(1, early[1]);

    // 6. Products: tiles 0 and 1 from registers, 2 and 3 from their slots as they land.
    auto product = [&](const uint4 (&a)[kRSteps][2]) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < kRSteps; ++j) {
            const i32x8 op = {static_cast<int>(a[j][0].x), static_cast<int>(a[j][0].y), static_cast<int>(a[j][0].z),
                              static_cast<int>(a[j][0].w), static_cast<int>(a[j][1].x), static_cast<int>(a[j][1].y),
                              static_cast<int>(a[j][1].z), static_cast<int>(a[j][1].w)};
            acc = mfma_f8(op, codes[j], acc);
        }
        return acc;
    };
    f32x4 acc[kRTiles];
    acc[0] = product(early[0]);
    acc[1] = product(early[1]);
#pragma unroll
    for (int t = 2; t < kRTiles; ++t) {
        __builtin_amdgcn_sched_barrier(0);  // the wait for tile t stays after the work above
        fence();
        if (t == 2) wait_vmcnt<kTileLoads>(); else wait_vmcnt<0>();
        fence();
        uint4 a[kRSteps][2];
        read_tile(t, a);
        acc[t] = product(a);
    }

    // 7. The waves' partial sums (over the slots, once every wave is done with its own), added
    //    in wave order; wave t finishes tile t.
    f32x4* part = reinterpret_cast<f32x4*>(slot0);  // [kRWaves][kRTiles][64]
    __syncthreads();
#pragma unroll
    for (int t = 0; t < kRTiles; ++t) part[(wave * kRTiles + t) * 64 + lane] = acc[t];
    __syncthreads();
    if (!emits) return;
    f32x4 sum = part[wave * 64 + lane];
#pragma unroll
    for (int w = 1; w < kRWaves; ++w) sum += part[(w * kRTiles + wave) * 64 + lane];
    uint32_t o[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float v = __fmul_rn(__fmul_rn(sum[i], s), wscale[i]);
        if constexpr (kBias) v = __fadd_rn(v, widen<kOutHalf>(bterm[i]));
        const uint32_t h = narrow<kOutHalf>(v);
        o[i / 2] = (i & 1) ? (o[i / 2] | (h << 16)) : h;
    }
    *reinterpret_cast<uint2*>(out + static_cast<int64_t>(r) * N + row0 + n_out) = make_uint2(o[0], o[1]);
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
// workgroup's rotation is shared by twice the rows); 6 (two workgroups a CU there) 9.0 -> 9.5 us
// and 8 slower.
constexpr int kIRows = 4;
// Activation registers a thread may hold (8 bf16 a uint4, 2048 elements a row a uint4 across the
// workgroup): 24, so that with the rotated values (M·K/256 floats) the widest admitted rows still
// fit one wave's 512 registers: M = 1 to K = 32768, M = 2 to 16384, M = 3 and 4 to 12288.
constexpr int kIXLoads = 24;

template <bool kXHalf, bool kOutHalf, bool kBias, int kM, int kChunks>
// (x is deliberately not __restrict__: loads through a read-only restrict argument count as
// invariant, and the compiler sank them below the weight stream into the blocks that use them,
// so the rotation's first wait, in-order, waited for every weight load of the batch.)
__global__ __launch_bounds__(kDThreads) void int8_decode_kernel(
    const uint16_t* x, const int8_t* __restrict__ W, const float* __restrict__ ws,
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
    const RowEpilogue<kIRows, kBias> epi = row_epilogue<kIRows, kBias>(ws, bias, nw, N);
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
            const float v = __fmul_rn(__fmul_rn(static_cast<float>(dot[i][m]), scale[m]), epi.ws[i]);
            uint32_t h = narrow<kOutHalf>(v);
            if constexpr (kBias)
                h = narrow<kOutHalf>(__fadd_rn(widen<kOutHalf>(static_cast<uint16_t>(h)), widen<kOutHalf>(epi.bias[i])));
            o[i / 2] = (i & 1) ? (o[i / 2] | (h << 16)) : h;
        }
        uint16_t* dst = out + static_cast<int64_t>(m) * N + nw;
        static_assert(kIRows == 4, "the store below writes four outputs");
        *reinterpret_cast<uint2*>(dst) = make_uint2(o[0], o[1]);
    }
}

// The int8 GEMV on codes already quantized (cozyq_gemm's int8 product at 1..4 rows, by the
// shape rule): int8_decode_kernel's weight stream, products and epilogue, with the rows' codes and
// scales read from memory instead of made in the workgroup. A thread loads 16-byte runs of every
// row (zeros past K) ahead of the weight stream and stores them to LDS, where the products read
// them as in the fused kernel; (acc·xs)·ws, one cast, + bias in the output dtype, as every tile.
template <bool kOutHalf, bool kBias, int kM, int kRuns>
// (q is not __restrict__, for int8_decode_kernel's reason: its loads must stay ahead of the
// weight stream.)
__global__ __launch_bounds__(kDThreads) void int8_codes_gemv_kernel(
    const int8_t* q, const float* xs, const int8_t* __restrict__ W, const float* __restrict__ ws,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int64_t ldo, int N, int K) {
    static_assert(kM * kRuns <= kIXLoads, "activation registers");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    int8_t* xq = reinterpret_cast<int8_t*>(smem);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int spans = (K + 1023) / 1024;
    const int stride = spans * 1024;
    const int nw = blockIdx.x * (kDWaves * kIRows) + wave * kIRows;  // the wave's first row

    // 1. The codes: the thread's 16-byte runs of every row, then the row scales and the
    // epilogue's operands, all ahead of the weight stream.
    uint4 cv[kM][kRuns];
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int8_t*>(q + static_cast<int64_t>(m) * K), 0, K, 0x00020000);
#pragma unroll
        for (int c = 0; c < kRuns; ++c)
            cv[m][c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(qr, c * (kDThreads * 16) + tid * 16, 0, 0));
    }
    float scale[kM];
#pragma unroll
    for (int m = 0; m < kM; ++m) scale[m] = xs[m];
    const RowEpilogue<kIRows, kBias> epi = row_epilogue<kIRows, kBias>(ws, bias, nw, N);
    asm volatile("" ::: "memory");  // the weight loads stay behind the codes'

    // 2. The weight stream, as int8_decode_kernel's.
    __amdgpu_buffer_rsrc_t wr[kIRows];
#pragma unroll
    for (int i = 0; i < kIRows; ++i)
        wr[i] = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int8_t*>(W + static_cast<int64_t>(min(nw + i, N - 1)) * K), 0, K, 0x00020000);
    constexpr bool kTwo = kRuns > 1;  // rows longer than one batch of spans
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

    // 3. The codes into LDS (`stride` bytes a row, zeros past K).
#pragma unroll
    for (int m = 0; m < kM; ++m)
#pragma unroll
        for (int c = 0; c < kRuns; ++c) {
            const int e = c * (kDThreads * 16) + tid * 16;
            if (e < stride) *reinterpret_cast<uint4*>(xq + m * stride + e) = cv[m][c];
        }
    __syncthreads();

    // 4. Products, the trace and the epilogue: int8_decode_kernel's.
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
        consume(wa, 0);
    }
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
            dot[i][m] = diagonal_sum(v);
        }
    if (lane != 0 || nw >= N) return;  // N % 4 == 0: a wave's rows are all in or all out
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        uint32_t o[(kIRows + 1) / 2];
#pragma unroll
        for (int i = 0; i < kIRows; ++i) {
            const float v = __fmul_rn(__fmul_rn(static_cast<float>(dot[i][m]), scale[m]), epi.ws[i]);
            uint32_t h = narrow<kOutHalf>(v);
            if constexpr (kBias)
                h = narrow<kOutHalf>(__fadd_rn(widen<kOutHalf>(static_cast<uint16_t>(h)), widen<kOutHalf>(epi.bias[i])));
            o[i / 2] = (i & 1) ? (o[i / 2] | (h << 16)) : h;
        }
        static_assert(kIRows == 4, "the store below writes four outputs");
        *reinterpret_cast<uint2*>(out + static_cast<int64_t>(m) * ldo + nw) = make_uint2(o[0], o[1]);
    }
}

template <bool kOutHalf, bool kBias>
hipError_t launch_int8_codes_gemv(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                                  const uint16_t* bias, uint16_t* out, int64_t ldo, int M, int N,
                                  int K, hipStream_t s) {
    const int blocks = (N + kDWaves * kIRows - 1) / (kDWaves * kIRows);
    const int64_t lds = static_cast<int64_t>(M) * ((K + 1023) / 1024) * 1024;
    const int runs = (K + kDThreads * 16 - 1) / (kDThreads * 16);
#define COZYQ_ROWS(R, C)                                                                           \
    if (M == R && runs <= C) {                                                                     \
        int8_codes_gemv_kernel<kOutHalf, kBias, R, C><<<blocks, kDThreads, lds, s>>>(q, xs, w, ws, bias, out, ldo, N, K); \
        return hipGetLastError();                                                                  \
    }
    COZYQ_ROWS(1, 1)
    COZYQ_ROWS(1, 3)
    COZYQ_ROWS(1, 8)
    COZYQ_ROWS(2, 1)
    COZYQ_ROWS(2, 4)
    COZYQ_ROWS(3, 1)
    COZYQ_ROWS(3, 3)
    COZYQ_ROWS(4, 1)
    COZYQ_ROWS(4, 3)
#undef COZYQ_ROWS
    return hipErrorNotSupported;
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

constexpr int kRowsMaxK = 128 * kRSpan;  // 4096
constexpr int64_t kRowsFromArea = 36864;  // rows x N from which 3 and 4 rows take the row tile
constexpr int kRowsWaves = 8;  // fp8_rows_kernel's waves a workgroup

template <bool kXHalf, bool kOutHalf, bool kBias>
hipError_t launch_rows(const uint16_t* x, const uint8_t* w, const float* ws, const uint16_t* bias,
                       uint16_t* out, int M, int N, int K, hipStream_t s) {
    int device = 0;
    const hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    const int units = N / 8;
    const int groups = max(min(cu_count(device), units), (units + 2 * kRTiles - 1) / (2 * kRTiles));
    fp8_rows_kernel<kXHalf, kOutHalf, kBias, kRowsWaves><<<groups, 64 * kRowsWaves, 0, s>>>(x, w, ws, bias, out, M, N, K, units, groups);
    return hipGetLastError();
}

}  // namespace

hipError_t fp8_linear_small(const void* x, bool x_half, const uint8_t* w, const float* ws,
                            const void* bias, void* out, bool out_half, int M, int N, int K,
                            hipStream_t s) {
    // 1..4 rows whose activation fits the registers (the GEMV), 5..16 rows with K <= 4096 (the
    // row-tile kernel); the rest is quantize + narrow GEMM. 3 and 4 rows of a wide weight also
    // take the row-tile kernel: each GEMV wave's MFMA chain grows with the rows, the row tile's
    // does not (graph replays over weights past the MALL, us GEMV / row tile: N=14336 K=4096
    // M=3 13.1 / 12.5, M=4 15.5 / 12.5; N=12288 K=3072 M=3 10.8 / 10.8, M=4 12.9 / 10.6;
    // N=4096 K=4096 M=4 6.8 / 9.5).
    const bool wide = M >= 3 && M <= 4 && static_cast<int64_t>(M) * N >= kRowsFromArea && K <= kRowsMaxK;
    const bool gemv = !wide && M >= 1 && M <= 4 && static_cast<int64_t>(M) * K <= kXLoads * kDThreads * 8;
    const bool tiles = wide || (M >= 5 && M <= 16 && K <= kRowsMaxK);
    if (!gemv && !tiles) return hipErrorNotSupported;
    auto xp = static_cast<const uint16_t*>(x);
    auto bp = static_cast<const uint16_t*>(bias);
    auto op = static_cast<uint16_t*>(out);
#define COZYQ_CASE(XH, OH, B)                                                                      \
    if (x_half == XH && out_half == OH && (bias != nullptr) == B)                                  \
        return gemv ? launch_decode<XH, OH, B>(xp, w, ws, bp, op, M, N, K, s)                      \
                    : launch_rows<XH, OH, B>(xp, w, ws, bp, op, M, N, K, s);
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

hipError_t int8_codes_gemv(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                           const void* bias, void* out, int64_t ldo, bool out_half, int M, int N,
                           int K, hipStream_t s) {
    // 1..4 rows whose codes fit the registers and 48 KiB of LDS: K <= 32768 at 1 row, 16384 at
    // 2, 12288 at 3..4. N % 4 == 0 (a wave's four rows all in or all out).
    if (M < 1 || M > 4 || N % 4 || K > (M == 1 ? 32768 : M == 2 ? 16384 : 12288)) return hipErrorNotSupported;
    auto bp = static_cast<const uint16_t*>(bias);
    auto op = static_cast<uint16_t*>(out);
    if (out_half)
        return bias ? launch_int8_codes_gemv<true, true>(q, xs, w, ws, bp, op, ldo, M, N, K, s)
                    : launch_int8_codes_gemv<true, false>(q, xs, w, ws, bp, op, ldo, M, N, K, s);
    return bias ? launch_int8_codes_gemv<false, true>(q, xs, w, ws, bp, op, ldo, M, N, K, s)
                : launch_int8_codes_gemv<false, false>(q, xs, w, ws, bp, op, ldo, M, N, K, s);
}

}  // namespace cozyq
