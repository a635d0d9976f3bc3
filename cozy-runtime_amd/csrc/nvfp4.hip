// The nvfp4 W4A16 GEMV on gfx950 (reference: the `_gemv` path of internal/nvfp4_linear.py:
// 126-201, served at most DECODE_ROWS = 16 rows, :338-377): out[m, n] = round((Σ_k x[m, k] ·
// bf16(e2m1[n, k] · s[n, k/16])) · g), float32 accumulation. The stored weight stays packed
// (0.56 bytes a weight): codes [N, K/2] (element 2k in the low nibble), E4M3 block scales in
// cuBLAS's 128x4 tiles (the leaf's resident layout), g the float32 second level.
//
// A workgroup of 8 waves takes 16 output rows (four rows from each 32-row quarter of a
// 128-row scale tile); wave w takes the 128-column macro steps w, w + 8,
// .... Per 32 columns a lane decodes 8 weights of its row: E2M1 by
// v_cvt_scalef32_pk_f32_fp4, times the E4M3 scale — exact in float32 and again in bf16 or fp16 —
// and one v_mfma_f32_16x16x32 multiplies them against the activation rows (zero past M).
// The eight waves' partial sums meet in LDS and are added in wave order, so a row's result does
// not depend on M or on the rows beside it. Every global read is a bounded buffer load: rows past
// N or M read zeros.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace cozyq {
namespace {

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2n __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2n __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2n __attribute__((ext_vector_type(2)));

constexpr int kGemvWaves = 8;
constexpr int kStepsAhead = 2;  // macro steps a wave keeps in flight

__device__ __forceinline__ __amdgpu_buffer_rsrc_t bounded_rsrc(const void* p, int64_t bytes) {
    const int64_t cap = bytes < 0x7fffffff ? bytes : 0x7fffffff;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(cap), 0x00020000);
}

// The eight weights of one code dword times the block scale, as the MFMA's packed operand. The
// conversion runs at scale 1 and the E4M3 scale multiplies after (exact in float32): the
// instruction's own scale operand is an MX exponent and keeps only a power of two.
template <bool kHalf>
__device__ __forceinline__ i32x4 weights8(uint32_t word, float s) {
    const int w = static_cast<int>(word);
    const f32x2n p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0) * s;
    const f32x2n p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1) * s;
    const f32x2n p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2) * s;
    const f32x2n p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3) * s;
    if constexpr (kHalf) {
        return i32x4{__builtin_bit_cast(int, __builtin_convertvector(p0, f16x2n)),
                     __builtin_bit_cast(int, __builtin_convertvector(p1, f16x2n)),
                     __builtin_bit_cast(int, __builtin_convertvector(p2, f16x2n)),
                     __builtin_bit_cast(int, __builtin_convertvector(p3, f16x2n))};
    } else {
        return i32x4{__builtin_bit_cast(int, __builtin_convertvector(p0, bf16x2n)),
                     __builtin_bit_cast(int, __builtin_convertvector(p1, bf16x2n)),
                     __builtin_bit_cast(int, __builtin_convertvector(p2, bf16x2n)),
                     __builtin_bit_cast(int, __builtin_convertvector(p3, bf16x2n))};
    }
}

// The two E4M3 block scales in the low 16 bits of `b`, as float32: the hardware conversion at
// scale 1 (exact, NaN for S.1111.111), with no branch.
__device__ __forceinline__ f32x2n scales2(uint32_t b) {
    return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(static_cast<int>(b), 1.0f, false);
}

template <bool kHalf>
__device__ __forceinline__ f32x4 mfma16(i32x4 a, i32x4 b, f32x4 c) {
    if constexpr (kHalf)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, a), __builtin_bit_cast(bf16x8v, b), c, 0, 0, 0);
}

// kXHalf: activations (and the weights fed beside them) fp16, else bf16; kOutHalf likewise.
// kMB: 16-row activation blocks (M ≤ 16·kMB), each its own MFMA against the same decoded weights.
// A macro step is 128 columns: a lane loads 16 bytes of its row's codes (32 weights, columns
// 128t + 32·sub ..), the two E4M3 scales that cover them (adjacent bytes of a 128x4 tile, as
// the first block is even) and, from each block, its activation row's 32 matching columns, and
// feeds 4 MFMAs a block, MFMA j taking columns 128t + 32·sub + 8j .. + 8 on both sides: every
// lane group pairs the same columns of A and B, so the four products add up to the 128-column
// dot product. A block's MFMAs and sums are the same whatever kMB is, so a row's result does
// not depend on M.
template <bool kXHalf, bool kOutHalf, int kMB>
__global__ __launch_bounds__(64 * kGemvWaves) void nvfp4_gemv_kernel(const uint16_t* __restrict__ x,
                                                                     const uint8_t* __restrict__ w,
                                                                     const uint8_t* __restrict__ scale,
                                                                     const float* __restrict__ scale_2,
                                                                     uint16_t* __restrict__ out, int M, int N, int K) {
    __shared__ f32x4 partial[kGemvWaves][kMB][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // A workgroup's 16 rows are 32q + 4j + p (q, p = 0..3) of a 128-row tile block: the four
    // 16-byte scale chunks of rows 4j .. 4j + 3 hold those 16 rows' scales, so a tile's bytes are
    // fetched once. MFMA row i is tile row 32·(i/4) + 4j + i%4.
    const int tile_block = blockIdx.x >> 3, j4 = 4 * (blockIdx.x & 7);
    const auto row_of = [&](int i) { return 128 * tile_block + 32 * (i >> 2) + j4 + (i & 3); };
    const int row = row_of(lane & 15);  // the weight row this lane decodes
    const int sub = lane >> 4;          // its 32-column quarter of a macro step
    const int width = K / 16, col_tiles = (width + 3) / 4;
    const __amdgpu_buffer_rsrc_t wr = bounded_rsrc(w, static_cast<int64_t>(N) * (K / 2));
    const __amdgpu_buffer_rsrc_t sr = bounded_rsrc(scale, static_cast<int64_t>((N + 127) / 128 * 128) * col_tiles * 4);
    const __amdgpu_buffer_rsrc_t xr = bounded_rsrc(x, static_cast<int64_t>(M) * K * 2);
    // Rows past N read past the codes' end (zeros); rows past M read past x's end (zeros).
    const int code_row = row < N ? row : N;
    int x_row[kMB];
#pragma unroll
    for (int b = 0; b < kMB; ++b) x_row[b] = 16 * b + (lane & 15) < M ? 16 * b + (lane & 15) : M;
    const int64_t code_base = static_cast<int64_t>(code_row) * (K / 2);
    const int tile_row = (row >> 7) * col_tiles, in_tile = (row & 31) * 16 + ((row & 127) >> 5) * 4;

    f32x4 acc[kMB];
#pragma unroll
    for (int b = 0; b < kMB; ++b) acc[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int macro = K / 128;  // whole macro steps; a 32..96-column tail is handled below
    for (int t0 = wave; t0 < macro; t0 += kGemvWaves * kStepsAhead) {
        i32x4 code[kStepsAhead], xv[kStepsAhead][kMB][4];
        uint32_t sbyte[kStepsAhead];
#pragma unroll
        for (int j = 0; j < kStepsAhead; ++j) {
            const int t = t0 + j * kGemvWaves;
            const bool live = t < macro;
            const int k = 128 * t + 32 * sub;
            const int b = k / 16;  // even
            code[j] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                wr, live ? static_cast<int>(code_base + k / 2) : 0x7ffffff0, 0, 0));
            const int sidx = row < N && live ? ((tile_row + (b >> 2)) * 512 + in_tile + (b & 3)) : 0x7ffffff0;
            sbyte[j] = __builtin_amdgcn_raw_buffer_load_b16(sr, sidx, 0, 0);
#pragma unroll
            for (int mb = 0; mb < kMB; ++mb) {
                const int xo = live ? static_cast<int>((static_cast<int64_t>(x_row[mb]) * K + k) * 2) : 0x7fffff00;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    xv[j][mb][q] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                        xr, xo + 16 * q, 0, 0));
            }
        }
#pragma unroll
        for (int j = 0; j < kStepsAhead; ++j) {
            const f32x2n sc = scales2(sbyte[j]);
            const float s0 = sc[0], s1 = sc[1];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const i32x4 wq = weights8<kXHalf>(static_cast<uint32_t>(code[j][q]), q < 2 ? s0 : s1);
#pragma unroll
                for (int mb = 0; mb < kMB; ++mb) acc[mb] = mfma16<kXHalf>(wq, xv[j][mb][q], acc[mb]);
            }
        }
    }
    // A tail of 1..3 32-column steps past the last whole macro step, one per wave.
    const int tail = (K % 128) / 32;
    if (wave < tail) {
        const int k = 128 * macro + 32 * wave + 8 * sub;
        const int b = k / 16;
        const uint32_t c = __builtin_amdgcn_raw_buffer_load_b32(wr, static_cast<int>(code_base + k / 2), 0, 0);
        const int sidx = row < N ? ((tile_row + (b >> 2)) * 512 + in_tile + (b & 3)) : 0x7fffffff;
        const uint32_t sb = __builtin_amdgcn_raw_buffer_load_b8(sr, sidx, 0, 0);
        const i32x4 wq = weights8<kXHalf>(c, e4m3_value(sb));
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb) {
            const i32x4 xt = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                xr, static_cast<int>((static_cast<int64_t>(x_row[mb]) * K + k) * 2), 0, 0));
            acc[mb] = mfma16<kXHalf>(wq, xt, acc[mb]);
        }
    }
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb) partial[wave][mb][lane] = acc[mb];
    __syncthreads();
    // Wave mb < kMB adds block mb's eight partial sums, in wave order.
    if (wave >= kMB) return;
    const int mb = wave;
    f32x4 sum = partial[0][mb][lane];
#pragma unroll
    for (int v = 1; v < kGemvWaves; ++v) {
        const f32x4 p = partial[v][mb][lane];
        sum = f32x4{sum[0] + p[0], sum[1] + p[1], sum[2] + p[2], sum[3] + p[3]};
    }
    // D[i][m]: lane holds MFMA rows 4·(lane/16) + r of column m = lane % 16.
    const float g = scale_2[0];
    const int m = 16 * mb + (lane & 15);
    if (m >= M) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int n = row_of(4 * (lane >> 4) + r);
        if (n < N) out[static_cast<int64_t>(m) * N + n] = narrow<kOutHalf>(sum[r] * g);
    }
}

// The row-block form for 5..64 rows (K % 128 == 0): a workgroup of 4 waves takes 64 weight rows,
// each wave 16 of them over all of K, so no partial sums meet; the activation's 16·kMB rows come
// through LDS in 512-column chunks (LDS-DMA, a ring of 3 up to 32 rows, else 2), read once per
// workgroup instead of once per wave, and a wave keeps kRowsAhead macro steps of its codes and
// scales in flight in registers.
// Per macro step a lane decodes its row's 32 weights (two E4M3 blocks) and feeds one MFMA per
// activation block, as the GEMV above does; a block's sums run in the same order for any kMB.
typedef __attribute__((address_space(3))) void GemvLds;
constexpr int kRowBlockFrom = 4;                  // rows above which the row-block form runs
constexpr int kChunkCols = 512;                   // activation columns a chunk
constexpr int kXRowBytes = 2 * kChunkCols + 16;   // one activation row of a chunk, padded
constexpr int kRowsAhead = 8;                     // macro steps of codes in flight a wave

template <int N>
__device__ __forceinline__ void gemv_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// One wave's share of a chunk's activation rows: row r (r % 4 == wave) is one 1 KiB load.
template <int kMB>
__device__ __forceinline__ void gemv_chunk(__amdgpu_buffer_rsrc_t xr, uint8_t* slot, int chunk, int M, int K,
                                           int wave, int lane) {
    const int col = chunk * (2 * kChunkCols) + 16 * lane;  // byte within a row
#pragma unroll
    for (int j = 0; j < 4 * kMB; ++j) {
        const int r = 4 * j + wave;
        const uint32_t off = (r < M && col < 2 * K) ? static_cast<uint32_t>(r * 2 * K + col) : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (GemvLds*)(slot + r * kXRowBytes), 16, off, 0, 0, 0);
    }
}

template <bool kXHalf, bool kOutHalf, int kMB>
__global__ __launch_bounds__(256) void nvfp4_rows_kernel(const uint16_t* __restrict__ x,
                                                         const uint8_t* __restrict__ w,
                                                         const uint8_t* __restrict__ scale,
                                                         const float* __restrict__ scale_2,
                                                         uint16_t* __restrict__ out, int M, int N, int K) {
    constexpr int kSlot = 16 * kMB * kXRowBytes;
    constexpr int kRing = kMB <= 2 ? 3 : 2;  // activation chunks in LDS (2 in flight when 3)
    __shared__ __attribute__((aligned(16))) uint8_t xs[kRing * kSlot];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int n0 = blockIdx.x * 64 + 16 * wave;  // the wave's first weight row
    const int row = n0 + (lane & 15);
    const int sub = lane >> 4;
    const int col_tiles = K / 64;
    const __amdgpu_buffer_rsrc_t wr = bounded_rsrc(w, static_cast<int64_t>(N) * (K / 2));
    const __amdgpu_buffer_rsrc_t sr = bounded_rsrc(scale, static_cast<int64_t>((N + 127) / 128 * 128) * col_tiles * 4);
    const __amdgpu_buffer_rsrc_t xr = bounded_rsrc(x, static_cast<int64_t>(M) * K * 2);
    // Rows past N read past the codes' end (zeros).
    const int64_t code_base = static_cast<int64_t>(row < N ? row : N) * (K / 2) + 16 * sub;
    const int tile_row = (row >> 7) * col_tiles, in_tile = (row & 31) * 16 + ((row & 127) >> 5) * 4;
    const int macro = K / 128, chunks = (macro + 3) / 4;

    i32x4 code[kRowsAhead];
    uint32_t sbyte[kRowsAhead];
    auto load = [&](int t, int slot) {  // past the last step: zeros, never used
        const bool live = t < macro;
        code[slot] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
            wr, live ? static_cast<int>(code_base + 64 * t) : 0x7ffffff0, 0, 0));
        const int b = 8 * t + 2 * sub;  // the first of its two blocks (even)
        const int sidx = row < N && live ? ((tile_row + (b >> 2)) * 512 + in_tile + (b & 3)) : 0x7ffffff0;
        sbyte[slot] = __builtin_amdgcn_raw_buffer_load_b16(sr, sidx, 0, 0);
    };

    f32x4 acc[kMB];
#pragma unroll
    for (int b = 0; b < kMB; ++b) acc[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // Issue order, per chunk: its activation DMA, then 8 code and scale loads; so at chunk c's
    // wait the loads issued after chunk c's DMA number 8 + (kRing - 2)·(4·kMB + 8).
    gemv_chunk<kMB>(xr, xs, 0, M, K, wave, lane);
#pragma unroll
    for (int t = 0; t < 4; ++t) load(t, t);
    if constexpr (kRing == 3) gemv_chunk<kMB>(xr, xs + kSlot, 1, M, K, wave, lane);
#pragma unroll
    for (int t = 4; t < kRowsAhead; ++t) load(t, t);

    // kRowsAhead / 4 chunks (the register window) an iteration, so that slots are static.
    constexpr int kWindowChunks = kRowsAhead / 4;
    for (int c0 = 0; c0 < chunks; c0 += kWindowChunks) {
#pragma unroll
        for (int h = 0; h < kWindowChunks; ++h) {
            const int c = c0 + h;
            // Chunk c landed (this wave's rows; the barrier makes every wave's visible), and
            // every wave is done with chunk c - 1's slot, which takes chunk c + kRing - 1.
            gemv_vmcnt<8 + (kRing - 2) * (4 * kMB + 8)>();
            __syncthreads();
            if (c >= chunks) break;
            gemv_chunk<kMB>(xr, xs + ((c + kRing - 1) % kRing) * kSlot, c + kRing - 1, M, K, wave, lane);
            const uint8_t* xc = xs + (c % kRing) * kSlot;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 4 * c + i, slot = 4 * h + i;
                if (t < macro) {
                    const f32x2n sc = scales2(sbyte[slot]);
                    const float s0 = sc[0], s1 = sc[1];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const i32x4 wq = weights8<kXHalf>(static_cast<uint32_t>(code[slot][q]), q < 2 ? s0 : s1);
#pragma unroll
                        for (int b = 0; b < kMB; ++b) {
                            const i32x4 xv = *reinterpret_cast<const i32x4*>(
                                xc + (16 * b + (lane & 15)) * kXRowBytes + 256 * i + 2 * (32 * sub + 8 * q));
                            acc[b] = mfma16<kXHalf>(wq, xv, acc[b]);
                        }
                    }
                }
                load(t + kRowsAhead, slot);
            }
        }
    }
    gemv_vmcnt<0>();  // the zero loads past the end land before the wave ends

    // D[i][m]: lane holds MFMA rows 4·(lane/16) + r of column m = lane % 16.
    const float g = scale_2[0];
    const int n = n0 + 4 * sub;
#pragma unroll
    for (int b = 0; b < kMB; ++b) {
        const int m = 16 * b + (lane & 15);
        if (m >= M) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (n + r < N) out[static_cast<int64_t>(m) * N + n + r] = narrow<kOutHalf>(acc[b][r] * g);
    }
}

// The streaming form for 1 or 2 activation rows and K ≤ 4096 (measured at config 3's weight: M = 1
// 11.7 → 8.9 µs, M = 2 12.0 → 11.5; from 3 rows the per-row MFMA chains make it slower than the
// K-split form): each wave streams kStreamRows whole
// weight rows as contiguous 1 KiB loads (lane l at byte 16·l of a 2 KiB span: its 32 codes,
// columns 2048·j + 32·l ..), with the non-temporal policy, the way the fp8 decode GEMV streams
// its rows, instead of 16 rows × 64 bytes an instruction. The activation rows sit in LDS (16-bit,
// zeros past K). MFMA q of a span takes each lane's 8 weights 8q .. 8q + 7 (decoded as the GEMV
// above does) as A row l%16, k-block l/16, and the activation's same 8 columns as B column l%16,
// so D[i][i] sums the 8-column products of the four lanes i, i + 16, i + 32, i + 48: the trace of
// D, accumulated over the four groups and the spans, is the row's dot product. One MFMA chain per
// activation row, so a row's result does not depend on M. The block scales of the workgroup's 8
// rows come into LDS first, by 16-byte loads of the 128-byte lines that hold them (a 128x4 tile
// keeps rows r .. r + 7 of a 32-row group in one line): a 2-byte load a lane and row touches 32
// lines an instruction and measured ~3 µs of config 3's M = 1 decode.
constexpr int kStreamWaves = 4;
constexpr int kStreamRows = 2;     // weight rows a wave streams
constexpr int kStreamBatch = 2;    // 2 KiB spans of each row in flight
constexpr int kStreamMaxK = 4096;  // activation rows a thread stages in registers: K ≤ this
constexpr int kStreamPolicy = 3;   // sc0 nt: each weight byte is read once per call
constexpr int kStreamRowsMax = 2;  // activation rows the streaming form serves

template <bool kXHalf, bool kOutHalf, int kM>
__global__ __launch_bounds__(64 * kStreamWaves) void nvfp4_stream_kernel(const uint16_t* __restrict__ x,
                                                                         const uint8_t* __restrict__ w,
                                                                         const uint8_t* __restrict__ scale,
                                                                         const float* __restrict__ scale_2,
                                                                         uint16_t* __restrict__ out, int N, int K) {
    extern __shared__ __attribute__((aligned(16))) uint8_t xl[];  // kM rows of `xbytes`, then the scales
    constexpr int kThreads = 64 * kStreamWaves;
    constexpr int kPieces = kStreamMaxK * 2 / 16 / kThreads;  // 16-byte activation pieces a thread, per row
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int spans = (K + 2047) / 2048, xbytes = spans * 4096;
    const int row0 = blockIdx.x * (kStreamWaves * kStreamRows);  // the workgroup's 8 rows
    const int n0 = row0 + wave * kStreamRows;
    const int width = K / 16, col_tiles = (width + 3) / 4;
    uint32_t* const sl = reinterpret_cast<uint32_t*>(xl + kM * xbytes);  // [span][8 rows][32 tiles]
    const __amdgpu_buffer_rsrc_t wr = bounded_rsrc(w, static_cast<int64_t>(N) * (K / 2));
    const __amdgpu_buffer_rsrc_t sr = bounded_rsrc(scale, static_cast<int64_t>((N + 127) / 128 * 128) * col_tiles * 4);
    const __amdgpu_buffer_rsrc_t xr = bounded_rsrc(x, static_cast<int64_t>(kM) * K * 2);

    // 1. The activation rows' pieces into registers first (a wave's loads complete in issue
    //    order: issued after the weights, they would wait for the whole stream).
    uint4 xv[kM][kPieces];
#pragma unroll
    for (int m = 0; m < kM; ++m)
#pragma unroll
        for (int p = 0; p < kPieces; ++p) {
            const int b = 16 * (tid + kThreads * p);  // byte within the row
            xv[m][p] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                xr, b < 2 * K ? m * 2 * K + b : 0x7ffffff0, 0, 0));
        }
    // The 8 rows' scale lines: thread t brings, for each span, the 16 bytes of column tile t/8
    // that hold row row0 + t%8 (and the three rows 32, 64 and 96 apart in its 128-row block).
    static_assert(kStreamWaves * kStreamRows == 8 && 64 * kStreamWaves == 256, "8 rows, 256 threads");
    uint4 svv[kStreamMaxK / 2048];
#pragma unroll
    for (int j = 0; j < kStreamMaxK / 2048; ++j) {
        const int tile = 32 * j + (tid >> 3), r = row0 + (tid & 7);
        const int off = ((r >> 7) * col_tiles + tile) * 512 + (r & 31) * 16;
        svv[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
            sr, j < spans && tile < col_tiles ? off : 0x7ffffff0, 0, 0));
    }
    asm volatile("" ::: "memory");

    // 2. The weight stream: kStreamBatch spans of each row.
    uint4 wv[kStreamRows][kStreamBatch];
    auto issue = [&](int first) {
#pragma unroll
        for (int i = 0; i < kStreamRows; ++i)
#pragma unroll
            for (int b = 0; b < kStreamBatch; ++b) {
                const int row = n0 + i, col = 2048 * (first + b) + 32 * lane;
                const bool live = row < N && col < K;
                wv[i][b] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                    wr, live ? row * (K / 2) + col / 2 : 0x7ffffff0, 0, kStreamPolicy));
            }
    };
    issue(0);

    // 3. The activation into LDS, zeros past K (the pieces past xbytes are never read).
#pragma unroll
    for (int m = 0; m < kM; ++m)
#pragma unroll
        for (int p = 0; p < kPieces; ++p) {
            const int b = 16 * (tid + kThreads * p);
            if (b < xbytes) *reinterpret_cast<uint4*>(xl + m * xbytes + b) = xv[m][p];
        }
    {
        // The row's dword of the 16 bytes: its 32-row group's slot (all 8 rows share it).
        const int slot = (row0 & 127) >> 5;
#pragma unroll
        for (int j = 0; j < kStreamMaxK / 2048; ++j) {
            const uint32_t d[4] = {svv[j].x, svv[j].y, svv[j].z, svv[j].w};
            if (j < spans) sl[(j * 8 + (tid & 7)) * 32 + (tid >> 3)] = d[slot];
        }
    }
    __syncthreads();

    // 4. Products: the trace accumulates over the groups and the spans.
    f32x4 acc[kStreamRows][kM];
#pragma unroll
    for (int i = 0; i < kStreamRows; ++i)
#pragma unroll
        for (int m = 0; m < kM; ++m) acc[i][m] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int first = 0; first < spans; first += kStreamBatch) {
        if (first != 0) issue(first);
#pragma unroll
        for (int b = 0; b < kStreamBatch; ++b) {
            if (first + b >= spans) break;
            i32x4 xb[kM][4];
#pragma unroll
            for (int m = 0; m < kM; ++m)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    xb[m][q] = *reinterpret_cast<const i32x4*>(xl + m * xbytes + 4096 * (first + b) + 64 * lane + 16 * q);
#pragma unroll
            for (int i = 0; i < kStreamRows; ++i) {
                // The lane's blocks 2l and 2l + 1 of the span: bytes 2(l&1) and 2(l&1) + 1 of tile l/2.
                const uint32_t sd = sl[((first + b) * 8 + wave * kStreamRows + i) * 32 + (lane >> 1)];
                const f32x2n sc = scales2(sd >> (16 * (lane & 1)));
                const uint32_t d[4] = {wv[i][b].x, wv[i][b].y, wv[i][b].z, wv[i][b].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const i32x4 wq = weights8<kXHalf>(d[q], q < 2 ? sc[0] : sc[1]);
#pragma unroll
                    for (int m = 0; m < kM; ++m) acc[i][m] = mfma16<kXHalf>(wq, xb[m][q], acc[i][m]);
                }
            }
        }
    }

    // 5. The trace: D[a][a] sits in lane a + 16·(a/4), register a % 4; the 64 lanes' sum.
    const int a = lane & 15;
    const bool diagonal = (lane >> 4) == (a >> 2);
    const float g = scale_2[0];
#pragma unroll
    for (int i = 0; i < kStreamRows; ++i)
#pragma unroll
        for (int m = 0; m < kM; ++m) {
            const f32x4 d = acc[i][m];
            const int r = a & 3;
            float v = r == 0 ? d[0] : (r == 1 ? d[1] : (r == 2 ? d[2] : d[3]));
            v = diagonal ? v : 0.0f;
            v = diagonal_sum(v);
            if (lane == 0 && n0 + i < N) out[static_cast<int64_t>(m) * N + n0 + i] = narrow<kOutHalf>(v * g);
        }
}

}  // namespace

hipError_t nvfp4_gemv(const void* x, bool x_half, const uint8_t* w, const uint8_t* scale, const float* scale_2,
                      void* out, bool out_half, int M, int N, int K, hipStream_t s) {
    const auto* xp = static_cast<const uint16_t*>(x);
    auto* op = static_cast<uint16_t*>(out);
    // More than 4 rows on a weight whose 64-row groups alone give 192 workgroups: the row-block
    // kernel (the activation read once per workgroup); otherwise the K-split GEMV.
    const bool rows = M > kRowBlockFrom && K % 128 == 0 && (N + 63) / 64 >= 192;
    // One or two rows of a short activation: the streaming form.
    if (M >= 1 && M <= kStreamRowsMax && K <= kStreamMaxK) {
        const int64_t lds = (static_cast<int64_t>(M) * 4096 + 1024) * ((K + 2047) / 2048);
        auto stream = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3((N + kStreamWaves * kStreamRows - 1) / (kStreamWaves * kStreamRows)),
                               dim3(64 * kStreamWaves), lds, s, xp, w, scale, scale_2, op, N, K);
            return hipGetLastError();
        };
        auto by_rows = [&](auto xh, auto oh) {
            constexpr bool kX = decltype(xh)::value, kO = decltype(oh)::value;
            return M == 1 ? stream(nvfp4_stream_kernel<kX, kO, 1>) : stream(nvfp4_stream_kernel<kX, kO, 2>);
        };
        using T = std::true_type;
        using F = std::false_type;
        if (x_half) return out_half ? by_rows(T{}, T{}) : by_rows(T{}, F{});
        return out_half ? by_rows(F{}, T{}) : by_rows(F{}, F{});
    }
    auto go = [&](auto kernel) {
        if (rows)
            hipLaunchKernelGGL(kernel, dim3((N + 63) / 64), dim3(256), 0, s, xp, w, scale, scale_2, op, M, N, K);
        else
            hipLaunchKernelGGL(kernel, dim3((N + 127) / 128 * 8), dim3(64 * kGemvWaves), 0, s, xp, w, scale, scale_2, op, M, N, K);
        return hipGetLastError();
    };
    auto blocks = [&](auto xh, auto oh) {
        constexpr bool kX = decltype(xh)::value, kO = decltype(oh)::value;
        switch ((M + 15) / 16 + (rows ? 4 : 0)) {
            case 1: return go(nvfp4_gemv_kernel<kX, kO, 1>);
            case 2: return go(nvfp4_gemv_kernel<kX, kO, 2>);
            case 3: return go(nvfp4_gemv_kernel<kX, kO, 3>);
            case 4: return go(nvfp4_gemv_kernel<kX, kO, 4>);
            case 5: return go(nvfp4_rows_kernel<kX, kO, 1>);
            case 6: return go(nvfp4_rows_kernel<kX, kO, 2>);
            case 7: return go(nvfp4_rows_kernel<kX, kO, 3>);
            case 8: return go(nvfp4_rows_kernel<kX, kO, 4>);
            default: return hipErrorInvalidValue;
        }
    };
    using T = std::true_type;
    using F = std::false_type;
    if (x_half) return out_half ? blocks(T{}, T{}) : blocks(T{}, F{});
    return out_half ? blocks(F{}, T{}) : blocks(F{}, F{});
}

}  // namespace cozyq
