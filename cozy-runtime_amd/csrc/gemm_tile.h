// The 256-row-tile GEMMs on gfx950 (256x256, or 256x192 columns): int8 W8A8 (exact int32 accumulation on
// v_mfma_i32_32x32x32_i8), fp8 e4m3 row-wise (v_mfma_scale_f32_32x32x64_f8f6f4, float32
// accumulation) and MXFP8 (the same MFMA with each operand's E8M0 block scales fed to the
// matrix core), with the dequantizing epilogue fused: out = epilogue(q · wᵀ), q [M, K] and
// w [N, K] with K contiguous, one byte an element. (Few-row GEMMs are gemm_narrow.hip.)
//
// A workgroup of 4 waves owns a 256x256 output tile (256x192: see gemm_tile); each wave a 128x128 quadrant as 4x4 MFMA
// blocks of 32x32 (256 accumulator registers a lane, held in AGPRs). A step's MFMAs consume 64
// bytes of K; the LDS holds two buffers of 128 bytes of K (the X and W tiles' 256 rows x 128
// bytes, and for MX their rows' four E8M0 bytes), so every load moves whole 128-byte cache lines
// (half-line loads measured 36% slower through L2 on MI355X). Buffers are filled by
// buffer_load ... lds straight from HBM/L2 — no staging registers, and rows past M or N and
// columns past K read as zeros through the buffer's bounds. A buffer is refilled two steps
// before it is read, one barrier every two steps; each step's MFMAs run on fragments read from
// LDS during the previous step. Tiles are ordered so that each XCD (workgroups b ≡ x mod 8)
// works through a contiguous run of tiles, 4 M-tiles by 8 N-tiles at a time, which share their
// X and W K-slices in that XCD's L2.
//
// MFMA rates from one wave per SIMD on MI355X: i8 32x32x32 82% of the int8 peak on low-entropy
// operands and 66% on random ones (power), f8 32x32x64 87%. The MFMA's A operand is the W tile
// and its B operand the X tile, so each lane's results are runs of four consecutive output
// columns of one row.
#pragma once

#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace cozyq {
namespace {

enum Kind { kInt8 = 0, kFp8 = 1, kMx = 2 };

constexpr int kTile = 256;
constexpr int kPairK = 128;                    // K bytes a buffer holds: two steps, whole lines
constexpr int kThreads = 256;
constexpr int kOpBytes = kTile * kPairK;       // one operand's buffer: 32 KB
constexpr int kScaleBytes = kTile * 4;         // MX: one operand's E8M0 bytes for a buffer
constexpr int kPairBytes = 2 * kOpBytes + 2 * kScaleBytes;  // X, W, X scales, W scales
constexpr uint32_t kOutOfRange = 0x80000000u;  // a buffer offset past num_records reads zeros
constexpr int kGroupM = 4;                     // M-tiles a tile group spans

constexpr int kStageRow = 128 * 2 + 16;         // one staged output row: 128 bf16 + pad
constexpr int kStageBytes = 128 * kStageRow;    // one wave's staged quadrant
constexpr int kEpiBase = 4 * kStageBytes > 2 * kPairBytes ? 4 * kStageBytes : 2 * kPairBytes;
// The tile's epilogue operands, loaded into LDS with the first buffer: 256 weight scales, 256
// biases and 256 row scales, past the buffers and the staging area.
constexpr int kWsOff = kEpiBase, kBiasOff = kEpiBase + 1024, kXsOff = kEpiBase + 1536;
constexpr int kLdsBytes = kEpiBase + 2560;

// Buffer loads a lane issues per buffer: 8 of 16 bytes for X, kTN / 32 for W, and for MX one
// of 4 bytes for each operand's scales.
template <int kKind, int kTN = 256>
constexpr int kLoads = 8 + kTN / 32 + (kKind == kMx ? 2 : 0);

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

// 16-byte chunk `c` (0..7) of a 128-byte LDS row `r` sits at chunk c ^ ((r/2) % 8): the 16 rows
// a ds_read_b128 serves together, read at one logical chunk, land on 16 distinct 16-byte bank
// groups of 256 bytes.
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two float32 values rounded to the output dtype (round to nearest even), packed low then high:
// bf16 pairs in one v_cvt_pk_bf16_f32, fp16 one by one through the fenced conversion.
template <bool kOutHalf>
__device__ __forceinline__ uint32_t round2(float a, float b) {
    if constexpr (kOutHalf) {
        return narrow<true>(a) | (static_cast<uint32_t>(narrow<true>(b)) << 16);
    } else {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
    }
}

template <bool kOutHalf>
__device__ __forceinline__ float low_of(uint32_t p) {
    if constexpr (kOutHalf) return widen<true>(static_cast<uint16_t>(p & 0xffff));
    return float_of(p << 16);
}

template <bool kOutHalf>
__device__ __forceinline__ float high_of(uint32_t p) {
    if constexpr (kOutHalf) return widen<true>(static_cast<uint16_t>(p >> 16));
    return float_of(p & 0xffff0000u);
}

// Two dequantized float32 values through the rest of the law: one rounding to the output
// dtype, + bias in that dtype (internal/int8_linear.py:276), then optionally tanh-GELU.
template <bool kOutHalf, bool kBias, int kEpi>
__device__ __forceinline__ uint32_t finish2(float a, float b, uint32_t bias2) {
    uint32_t p = round2<kOutHalf>(a, b);
    if constexpr (kBias)
        p = round2<kOutHalf>(__fadd_rn(low_of<kOutHalf>(p), low_of<kOutHalf>(bias2)),
                             __fadd_rn(high_of<kOutHalf>(p), high_of<kOutHalf>(bias2)));
    if constexpr (kEpi == 1)
        p = round2<kOutHalf>(gelu_tanh(low_of<kOutHalf>(p)), gelu_tanh(high_of<kOutHalf>(p)));
    return p;
}

// Two float32 values of the fp8 / MX laws (bias already added in float32) through the rest of
// the epilogue: one rounding to the output dtype, then optionally tanh-GELU.
template <bool kOutHalf, int kEpi>
__device__ __forceinline__ uint32_t finish2_float(float a, float b) {
    uint32_t p = round2<kOutHalf>(a, b);
    if constexpr (kEpi == 1)
        p = round2<kOutHalf>(gelu_tanh(low_of<kOutHalf>(p)), gelu_tanh(high_of<kOutHalf>(p)));
    return p;
}

// One step's operands a lane holds: 4 W-row and 4 X-row fragments of 32 bytes (16-byte chunks
// g and g+2 of the step's 64 bytes for lane group g = l/32: the int8 MFMA takes them as two K
// halves, the f8f6f4 MFMA as one K = 64 operand), and for MX the E8M0 byte of each fragment's
// K block g.
struct Frags {
    i32x8 a[4], b[4];
    int sa[4], sb[4];
};

__device__ __forceinline__ i32x4 half_of(const i32x8& v, int h) {
    return h == 0 ? __builtin_shufflevector(v, v, 0, 1, 2, 3) : __builtin_shufflevector(v, v, 4, 5, 6, 7);
}

// One 256 x kTN output tile (tm, tn) by the workgroup's 4 waves, `lds` holding kLdsBytes. The
// caller has made sure every wave is done with `lds` from any earlier use. kEpi: 0 the law's
// dequantization (+ bias), 1 that then tanh-GELU, 2 the raw int32 accumulators (int8 test
// entry). kTN is 256, or 192: each wave then owns 128 x 96 (3 x 4 blocks), for grids that 256
// columns would leave a partial round of tiles (N = 3072: 256 tiles of 256 x 192 at M = 4096
// against 192 of 256 x 256); or 128 (2 x 4 blocks), the half-width tiles a grid's partial last
// round runs as. Each output's K sum runs in the same MFMA order every way.
template <int kKind, bool kOutHalf, bool kBias, int kEpi, int kTN = 256>
__device__ __forceinline__ void gemm_tile(
    uint8_t* __restrict__ lds, const uint8_t* __restrict__ X, const uint8_t* __restrict__ W,
    const float* __restrict__ xs, const float* __restrict__ ws, const uint8_t* __restrict__ xe,
    const uint8_t* __restrict__ we, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out,
    int32_t* __restrict__ acc_out, int64_t ldo, int M, int N, int K, int tm, int tn) {
    static_assert(kEpi != 2 || kKind == kInt8, "raw accumulators are the int8 GEMM's");
    static_assert(kTN == 256 || kTN == 192 || kTN == 128, "tile widths: 256, 192 or 128 columns");
    typedef std::conditional_t<kKind == kInt8, i32x16, f32x16> Acc;
    constexpr int kNI = kTN / 64;      // W blocks of 32 columns a wave
    constexpr int kHalfN = kTN / 2;    // a wave's columns
    constexpr int kWLoads = kTN / 32;  // W buffer loads a wave

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS-DMA bases go in M0
    const int wm = wave >> 1, wn = wave & 1;

    // The tile arithmetic divides on the vector unit; the origin is uniform, and buffer
    // descriptors must sit in scalar registers.
    const int m0 = __builtin_amdgcn_readfirstlane(tm * kTile);
    const int n0 = __builtin_amdgcn_readfirstlane(tn * kTN);

    // Buffer views of this tile's rows: reads past the last row return zeros.
    auto rows_view = [&](const uint8_t* base, int rows_left, int row_bytes) {
        const int64_t span = static_cast<int64_t>(rows_left) * row_bytes;
        const uint32_t bytes = span > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(span);
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, bytes, 0x00020000);
    };
    const __amdgpu_buffer_rsrc_t xr = rows_view(X + static_cast<int64_t>(m0) * K, M - m0, K);
    const __amdgpu_buffer_rsrc_t wr = rows_view(W + static_cast<int64_t>(n0) * K, N - n0, K);
    const int kb = K / 32;  // MX: E8M0 bytes a row (K % 128 == 0)
    __amdgpu_buffer_rsrc_t xer = xr, wer = wr;
    if constexpr (kKind == kMx) {
        xer = rows_view(xe + static_cast<int64_t>(m0) * kb, M - m0, kb);
        wer = rows_view(we + static_cast<int64_t>(n0) * kb, N - n0, kb);
    }
    const int soff = (64 * wave + lane) * kb;  // MX: the lane's scale row in the tile

    // Load j (0..7) of a wave fills LDS rows [(4j + wave)·8, +8) of an operand's buffer: lane l
    // writes row +l/8, physical chunk l%8 (whole 128-byte lines, 8 lanes a row), so it reads that
    // row's logical chunk (l%8) ^ swz. MX scales: wave w's lane l loads the four E8M0 bytes of
    // row 64w + l.
    int rowoff[8], chunk[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int r = (4 * j + wave) * 8 + (lane >> 3);
        chunk[j] = 16 * swz(r, lane & 7);
        rowoff[j] = r * K + chunk[j];
    }
#define COZYQ_ISSUE(pair)                                                                            \
    do {                                                                                             \
        uint8_t* buf_ = lds + ((pair) & 1) * kPairBytes;                                             \
        const int k0_ = (pair) * kPairK;                                                             \
        _Pragma("unroll") for (int j = 0; j < 8; ++j) {                                              \
            const uint32_t off_ = (k0_ + chunk[j] < K) ? static_cast<uint32_t>(rowoff[j] + k0_) : kOutOfRange; \
            const int base_ = (4 * j + wave) * 1024;                                                 \
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (LdsPtr*)(buf_ + base_), 16, off_, 0, 0, 0); \
            if (j < kWLoads)                                                                         \
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (LdsPtr*)(buf_ + kOpBytes + base_), 16, off_, 0, 0, 0); \
        }                                                                                            \
        if constexpr (kKind == kMx) {                                                                \
            const uint32_t so_ = (4 * (pair) < kb) ? static_cast<uint32_t>(soff + 4 * (pair)) : kOutOfRange; \
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xer, (LdsPtr*)(buf_ + 2 * kOpBytes + 256 * wave), 4, so_, 0, 0, 0); \
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wer, (LdsPtr*)(buf_ + 2 * kOpBytes + kScaleBytes + 256 * wave), 4, so_, 0, 0, 0); \
        }                                                                                            \
    } while (0)

    // Fragment reads (lane l supplies row l%32; lane group l/32 its K chunks): A = W rows (wn
    // half), B = X rows (wm half); step e (0, 1) of a buffer reads its logical chunks 4e + 2h +
    // l/32, h = 0, 1, and (MX) byte 2e + l/32 of the row's four scale bytes.
    const int fr = lane & 31, fq = lane >> 5;
    int aoff[2][2][4], boff[2][2][4];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rw = wn * kHalfN + min(i, kNI - 1) * 32 + fr, rx = wm * 128 + i * 32 + fr;
                aoff[e][h][i] = kOpBytes + rw * kPairK + 16 * swz(rw, 4 * e + 2 * h + fq);
                boff[e][h][i] = rx * kPairK + 16 * swz(rx, 4 * e + 2 * h + fq);
            }
    // Step s reads buffer (s/2) % 2, half s % 2.
    auto fetch = [&](int step, Frags& f) {
        const uint8_t* buf = lds + ((step >> 1) & 1) * kPairBytes;
        const int e = step & 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i < kNI) {
                const i32x4 alo = *reinterpret_cast<const i32x4*>(buf + aoff[e][0][i]);
                const i32x4 ahi = *reinterpret_cast<const i32x4*>(buf + aoff[e][1][i]);
                f.a[i] = __builtin_shufflevector(alo, ahi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
            const i32x4 blo = *reinterpret_cast<const i32x4*>(buf + boff[e][0][i]);
            const i32x4 bhi = *reinterpret_cast<const i32x4*>(buf + boff[e][1][i]);
            f.b[i] = __builtin_shufflevector(blo, bhi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
        if constexpr (kKind == kMx) {
            const int shift = 8 * (2 * e + fq);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (i < kNI) {
                    const int rw = wn * kHalfN + i * 32 + fr;
                    const uint32_t sw = *reinterpret_cast<const uint32_t*>(buf + 2 * kOpBytes + kScaleBytes + 4 * rw);
                    f.sa[i] = static_cast<int>((sw >> shift) & 0xff);
                }
                const int rx = wm * 128 + i * 32 + fr;
                const uint32_t sx = *reinterpret_cast<const uint32_t*>(buf + 2 * kOpBytes + 4 * rx);
                f.sb[i] = static_cast<int>((sx >> shift) & 0xff);
            }
        }
    };

    Acc acc[kNI][4];
#pragma unroll
    for (int i = 0; i < kNI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    const int np = (K + kPairK - 1) / kPairK;
    // Buffers 0 and 1 take pairs 0 and 1; pair p + 2 is issued at the top of step 2p + 1, once
    // every wave's reads of pair p are in registers, and must land by the top of step 2p + 3.
    // Past the last pair the offsets fall outside the buffer: zeros into a buffer nothing reads.
    // The epilogue's operands first (they land before pair 0 is seen complete): wave w loads
    // columns (rows) 64w..64w+63 of the tile; past N (M) they read as zeros.
    if constexpr (kEpi != 2) {
        const int c = 64 * wave + lane;
        if constexpr (kKind != kMx) {
            const auto wsr = rows_view(reinterpret_cast<const uint8_t*>(ws + n0), N - n0, 4);
            const auto xsr = rows_view(reinterpret_cast<const uint8_t*>(xs + m0), M - m0, 4);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wsr, (LdsPtr*)(lds + kWsOff + 256 * wave), 4, 4 * c, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xsr, (LdsPtr*)(lds + kXsOff + 256 * wave), 4, 4 * c, 0, 0, 0);
        }
        // Biases two a lane (LDS-DMA writes each lane's data at a 4-byte stride whatever the
        // load size): waves 0 and 1 cover the tile's 256.
        if constexpr (kBias) {
            if (wave < 2) {
                const auto br = rows_view(reinterpret_cast<const uint8_t*>(bias + n0), N - n0, 2);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(br, (LdsPtr*)(lds + kBiasOff + 256 * wave), 4, 4 * c, 0, 0, 0);
            }
        }
    }
    COZYQ_ISSUE(0);
    COZYQ_ISSUE(1);
    fence();
    wait_vmcnt<kLoads<kKind, kTN>>();  // pair 0 complete
    __builtin_amdgcn_s_barrier();
    fence();

    Frags f0, f1;
    fetch(0, f0);

    auto mfmas = [&](const Frags& c) {
        if constexpr (kKind == kInt8) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < kNI; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(half_of(c.a[i], h), half_of(c.b[j], h), acc[i][j], 0, 0, 0);
        } else {
#pragma unroll
            for (int i = 0; i < kNI; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (kKind == kMx)
                        acc[i][j] = mfma_f8_32_scaled(c.a[i], c.b[j], acc[i][j], c.sa[i], c.sb[j]);
                    else
                        acc[i][j] = mfma_f8_32(c.a[i], c.b[j], acc[i][j]);
                }
        }
    };
    // Issue order within a step: LDS reads spread one (MX: one to two) per MFMA group. A step
    // has 4·kNI MFMA groups and 2·(kNI + 4) fragment reads (MX: and kNI + 4 scale reads); the
    // reads past the groups (192 columns: 2, MX 3) follow them.
    auto schedule = [&]() {
        if constexpr (kKind == kInt8) {
#pragma unroll
            for (int g = 0; g < 4 * kNI; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // 2 MFMA
            }
        } else if constexpr (kKind == kFp8) {
#pragma unroll
            for (int g = 0; g < 4 * kNI; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
        } else {
#pragma unroll
            for (int g = 0; g < 2 * kNI; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
        }
        // The reads past the groups: 2·(kNI + 4) fragment reads (MX: and kNI + 4 scale reads)
        // against one a group (MX: three a pair of groups).
        if constexpr (kTN != 256) __builtin_amdgcn_sched_group_barrier(0x100, kKind == kMx ? 12 - 3 * kNI : 8 - 2 * kNI, 0);
    };
    // Step 2p: the next step's fragments come from the same buffer, which has landed.
    auto even_step = [&](int s, const Frags& cur, Frags& next) {
        fetch(s + 1, next);
        mfmas(cur);
        schedule();
    };
    // Step 2p + 1: pair p + 1 must have landed (the only loads in flight), every wave's reads of
    // pair p are done, and its buffer takes pair p + 2.
    auto odd_step = [&](int s, const Frags& cur, Frags& next) {
        fence();
        wait_vmcnt<0>();
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();
        fence();
        COZYQ_ISSUE((s >> 1) + 2);
        fetch(s + 1, next);  // past the last step: unused registers
        mfmas(cur);
        __builtin_amdgcn_sched_group_barrier(0x020, kLoads<kKind, kTN>, 0);  // the buffer loads first
        schedule();
    };
    for (int s = 0; s < 2 * np; s += 2) {
        even_step(s, f0, f1);
        odd_step(s + 1, f1, f0);
    }

    // Epilogue. Block (i, j): lane holds out[m][n] for m = j-block row l%32 and, per register
    // r, n = i-block column 8·(r/4) + 4·(l/32) + r%4 (MFMA rows are W rows): four runs of four
    // consecutive columns, each an 8-byte store. The lane's 64 weight scales and biases and 4
    // row scales are read from LDS once, ahead of the arithmetic.
    const int nl = n0 + wn * kHalfN + 4 * fq;  // the lane's first column
    if constexpr (kEpi == 2) {
        wait_vmcnt<0>();  // the zero-filling loads past the last step land before the LDS is released
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = m0 + wm * 128 + j * 32 + fr;
            if (m >= M) continue;
#pragma unroll
            for (int i = 0; i < kNI; ++i)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int n = nl + i * 32 + 8 * g;
                    if (n < N)
                        *reinterpret_cast<i32x4*>(acc_out + static_cast<int64_t>(m) * N + n) =
                            i32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                }
        }
        return;
    }
    // All loads have landed and all waves are done with the buffers before they become the
    // staging area.
    fence();
    wait_vmcnt<0>();
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    fence();
    float4 wsv[kNI][4];
    uint2 bv[kNI][4];
#pragma unroll
    for (int i = 0; i < kNI; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int c = nl - n0 + i * 32 + 8 * g;  // column within the tile
            wsv[i][g] = kKind == kMx ? make_float4(1.0f, 1.0f, 1.0f, 1.0f)
                                     : *reinterpret_cast<const float4*>(lds + kWsOff + 4 * c);
            if constexpr (kBias) bv[i][g] = *reinterpret_cast<const uint2*>(lds + kBiasOff + 2 * c);
        }
    float xsv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        xsv[j] = kKind == kMx ? 1.0f : *reinterpret_cast<const float*>(lds + kXsOff + 4 * (wm * 128 + j * 32 + fr));
    // Block row j at a time: its 32 rows are computed and staged, then stored as whole rows while
    // the next block row's arithmetic runs (the stores are not waited on).
    uint8_t* stage = lds + wave * kStageBytes;
    const int cl = (lane & 15) * 8;  // first of the lane's 8 columns in a stored row
    const int n = n0 + wn * kHalfN + cl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ml = j * 32 + fr;  // row within the quadrant
#pragma unroll
        for (int i = 0; i < kNI; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float w4[4] = {wsv[i][g].x, wsv[i][g].y, wsv[i][g].z, wsv[i][g].w};
                const uint2 b2 = kBias ? bv[i][g] : make_uint2(0, 0);
                uint2 packed;
                if constexpr (kKind == kInt8) {
                    // internal/int8_linear.py:445-448: (acc·xs)·ws, each product rounded to float32.
                    float v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        v[r] = __fmul_rn(__fmul_rn(static_cast<float>(acc[i][j][4 * g + r]), xsv[j]), w4[r]);
                    packed = make_uint2(finish2<kOutHalf, kBias, kEpi>(v[0], v[1], b2.x),
                                        finish2<kOutHalf, kBias, kEpi>(v[2], v[3], b2.y));
                } else {
                    // internal/fp8_linear.py:92-111 (`_scaled_mm` with row and column scales):
                    // (acc·xs)·ws (MX: acc, its block scales applied in the MFMA), + bias in float32.
                    float v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        v[r] = acc[i][j][4 * g + r];
                        if constexpr (kKind == kFp8) v[r] = __fmul_rn(__fmul_rn(v[r], xsv[j]), w4[r]);
                    }
                    if constexpr (kBias) {
                        v[0] = __fadd_rn(v[0], low_of<kOutHalf>(b2.x));
                        v[1] = __fadd_rn(v[1], high_of<kOutHalf>(b2.x));
                        v[2] = __fadd_rn(v[2], low_of<kOutHalf>(b2.y));
                        v[3] = __fadd_rn(v[3], high_of<kOutHalf>(b2.y));
                    }
                    packed = make_uint2(finish2_float<kOutHalf, kEpi>(v[0], v[1]),
                                        finish2_float<kOutHalf, kEpi>(v[2], v[3]));
                }
                const int col = i * 32 + 8 * g + 4 * fq;  // column within the quadrant
                *reinterpret_cast<uint2*>(stage + ml * kStageRow + 2 * col) = packed;
            }
        wait_lgkmcnt0();  // a wave reads back only its own rows
        // Whole rows: 16 lanes cover one quadrant row's 256 bytes (kHalfN = 96: the first 12 of
        // them, 192 bytes); 4 rows an instruction.
#pragma unroll
        for (int r0 = 0; r0 < 32; r0 += 4) {
            const int rl = j * 32 + r0 + (lane >> 4);
            const int m = m0 + wm * 128 + rl;
            const uint4 v = *reinterpret_cast<const uint4*>(stage + rl * kStageRow + 2 * cl);
            if (m < M && n < N && cl < kHalfN) *reinterpret_cast<uint4*>(out + static_cast<int64_t>(m) * ldo + n) = v;
        }
    }
}

// The tile order of one launch: XCD-contiguous runs (workgroup b runs on XCD b mod 8), then
// groups of kGroupM M-tiles with N fastest inside, so an XCD's concurrent tiles share their X
// and W K-slices in its L2.
__device__ __forceinline__ int2 launch_tile(int b, int tiles_m, int tiles_n) {
    const int tiles = tiles_m * tiles_n;
    int t = b;
    if ((tiles & 7) == 0) t = (t & 7) * (tiles >> 3) + (t >> 3);
    const int group = t / (kGroupM * tiles_n);
    const int gm = min(kGroupM, tiles_m - group * kGroupM);
    const int within = t - group * kGroupM * tiles_n;
    return make_int2(group * kGroupM + within % gm, within / gm);
}

template <int kKind, bool kOutHalf, bool kBias, int kEpi, int kTN = 256>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(
    const uint8_t* __restrict__ X, const uint8_t* __restrict__ W, const float* __restrict__ xs,
    const float* __restrict__ ws, const uint8_t* __restrict__ xe, const uint8_t* __restrict__ we,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int32_t* __restrict__ acc_out,
    int64_t ldo, int M, int N, int K, int tiles_m, int tiles_n) {
    // The two buffers during the K loop; afterwards each wave's 128x128 output quadrant, staged
    // for whole-row stores (rows padded to kStageRow bytes).
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kLdsBytes];
    const int2 t = launch_tile(blockIdx.x, tiles_m, tiles_n);
    gemm_tile<kKind, kOutHalf, kBias, kEpi, kTN>(lds, X, W, xs, ws, xe, we, bias, out, acc_out, ldo, M, N, K, t.x, t.y);
}

#undef COZYQ_ISSUE

// ---------------------------------------------------------------- int8 256x256 with 8 waves
//
// The int8 and fp8 256x256 tiles with the law's epilogue run as 8 waves, two a SIMD: wave w owns X rows
// 128·(w/4).. (4 blocks of 32) and W rows 64·(w%4).. (2 blocks), 128 accumulators, so two waves
// fit a SIMD's registers. A SIMD's second wave issues while the first waits (on LDS reads, the
// pair barrier) and the epilogue's VALU work comes from both: C2 (4096 x 12288 x 3072, bias +
// GELU) 168-170 -> 155-156 us on one box, outputs bit-identical to the 4-wave tile (int32 sums
// are exact in any order). Each wave reads 1.5x the fragment bytes a 4-wave quadrant does per
// MFMA, within the LDS's rate. Fragments are fetched a K half (32 bytes) at a time, one half
// ahead, so the two halves' registers and the accumulators stay within 256.
constexpr int kThreads8 = 512;
constexpr int kStageRow8 = 64 * 2 + 16;                 // staged output row: 64 outputs + pad
constexpr int kStageBytes8 = 128 * kStageRow8;          // one wave's staged 128 x 64
constexpr int kEpiBase8 = 8 * kStageBytes8 > 2 * kPairBytes ? 8 * kStageBytes8 : 2 * kPairBytes;
constexpr int kWsOff8 = kEpiBase8, kBiasOff8 = kEpiBase8 + 1024, kXsOff8 = kEpiBase8 + 1536;
constexpr int kLdsBytes8 = kEpiBase8 + 2560;
constexpr int kLoads8 = 8;                              // LDS-DMA loads a wave a pair (4 X, 4 W)
static_assert(kLdsBytes8 <= 160 * 1024, "one workgroup's LDS");

template <int kKind, bool kOutHalf, bool kBias, int kEpi>
__device__ __forceinline__ void gemm_tile8(
    uint8_t* __restrict__ lds, const uint8_t* __restrict__ X, const uint8_t* __restrict__ W,
    const float* __restrict__ xs, const float* __restrict__ ws, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ out, int64_t ldo, int M, int N, int K, int tm, int tn) {
    static_assert(kEpi == 0 || kEpi == 1, "the law's epilogue, optionally tanh-GELU");
    static_assert(kKind == kInt8 || kKind == kFp8, "int8 and fp8 (MX keeps the 4-wave tile)");
    typedef std::conditional_t<kKind == kInt8, i32x16, f32x16> Acc;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    const int m0 = __builtin_amdgcn_readfirstlane(tm * kTile);
    const int n0 = __builtin_amdgcn_readfirstlane(tn * kTile);
    auto rows_view = [&](const uint8_t* base, int rows_left, int row_bytes) {
        const int64_t span = static_cast<int64_t>(rows_left) * row_bytes;
        const uint32_t bytes = span > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(span);
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, bytes, 0x00020000);
    };
    const __amdgpu_buffer_rsrc_t xr = rows_view(X + static_cast<int64_t>(m0) * K, M - m0, K);
    const __amdgpu_buffer_rsrc_t wr = rows_view(W + static_cast<int64_t>(n0) * K, N - n0, K);

    // Load j (0..3) of a wave fills rows [(8j + wave)·8, +8) of each operand's buffer, whole
    // 128-byte lines as the 4-wave tile's loads do.
    int rowoff[4], chunk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = (8 * j + wave) * 8 + (lane >> 3);
        chunk[j] = 16 * swz(r, lane & 7);
        rowoff[j] = r * K + chunk[j];
    }
    auto issue = [&](int pair) {
        uint8_t* buf = lds + (pair & 1) * kPairBytes;
        const int k0 = pair * kPairK;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t off = (k0 + chunk[j] < K) ? static_cast<uint32_t>(rowoff[j] + k0) : kOutOfRange;
            const int base = (8 * j + wave) * 1024;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (LdsPtr*)(buf + base), 16, off, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (LdsPtr*)(buf + kOpBytes + base), 16, off, 0, 0, 0);
        }
    };

    // int8: half q = 2·step + h reads the buffer's chunks 4e + 2h + l/32 (e the step's parity;
    // step s reads buffer (s/2) % 2), one 32-byte K half of the i8 MFMA. fp8: a step's 64 bytes
    // (chunks 4e + l/32 and 4e + 2 + l/32: the f8 MFMA's K = 64 operand) in two pieces, W blocks
    // with X blocks 0-1, then X blocks 2-3 on the same W fragments.
    const int fr = lane & 31, fq = lane >> 5;
    auto frag_at = [&](int step, int h, bool w_side, int block) {
        const uint8_t* buf = lds + ((step >> 1) & 1) * kPairBytes + (w_side ? kOpBytes : 0);
        const int row = w_side ? wn * 64 + block * 32 + fr : wm * 128 + block * 32 + fr;
        return *reinterpret_cast<const i32x4*>(buf + row * kPairK + 16 * swz(row, 4 * (step & 1) + 2 * h + fq));
    };
    auto frag8_at = [&](int step, bool w_side, int block) {
        const i32x4 lo = frag_at(step, 0, w_side, block), hi = frag_at(step, 1, w_side, block);
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };

    Acc acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    // The epilogue's operands first (waves 0-3 cover the tile's 256 columns and rows).
    if (wave < 4) {
        const int c = 64 * wave + lane;
        const auto wsr = rows_view(reinterpret_cast<const uint8_t*>(ws + n0), N - n0, 4);
        const auto xsr = rows_view(reinterpret_cast<const uint8_t*>(xs + m0), M - m0, 4);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wsr, (LdsPtr*)(lds + kWsOff8 + 256 * wave), 4, 4 * c, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xsr, (LdsPtr*)(lds + kXsOff8 + 256 * wave), 4, 4 * c, 0, 0, 0);
        if constexpr (kBias) {
            if (wave < 2) {
                const auto br = rows_view(reinterpret_cast<const uint8_t*>(bias + n0), N - n0, 2);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(br, (LdsPtr*)(lds + kBiasOff8 + 256 * wave), 4, 4 * c, 0, 0, 0);
            }
        }
    }
    const int np = (K + kPairK - 1) / kPairK;
    issue(0);
    issue(1);
    fence();
    wait_vmcnt<kLoads8>();  // pair 0 (and the epilogue operands ahead of it) complete
    __builtin_amdgcn_s_barrier();
    fence();
    // Pair p: before its last piece, pair p + 1 must have landed and every wave's reads of pair
    // p be done: the workgroup meets, pair p + 2 refills buffer p % 2, and the next piece comes
    // from buffer (p + 1) % 2. Past the last pair the loads read zeros into a buffer nothing reads.
    auto meet = [&](int p) {
        fence();
        wait_vmcnt<0>();
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();
        fence();
        issue(p + 2);
    };
    __builtin_amdgcn_s_setprio(1);
    if constexpr (kKind == kInt8) {
        struct Half { i32x4 a[2], b[4]; };
        auto fetch = [&](int q, Half& f) {
#pragma unroll
            for (int i = 0; i < 2; ++i) f.a[i] = frag_at(q >> 1, q & 1, true, i);
#pragma unroll
            for (int j = 0; j < 4; ++j) f.b[j] = frag_at(q >> 1, q & 1, false, j);
        };
        auto mfmas = [&](const Half& c) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(c.a[i], c.b[j], acc[i][j], 0, 0, 0);
        };
        Half f0, f1;
        fetch(0, f0);
        for (int p = 0; p < np; ++p) {
            const int q = 4 * p;
            fetch(q + 1, f1);
            mfmas(f0);
            fetch(q + 2, f0);
            mfmas(f1);
            fetch(q + 3, f1);
            mfmas(f0);
            meet(p);
            fetch(q + 4, f0);
            mfmas(f1);
        }
    } else {
        // W fragments of two steps alternate (wa0 for even steps, wa1 for odd); xb holds the X
        // blocks of the piece running, xn those fetched for the next.
        i32x8 wa0[2], wa1[2], xb[2], xn[2];
        auto mfmas = [&](const i32x8 (&a)[2], const i32x8 (&b)[2], int j0) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j0 + j] = mfma_f8_32(a[i], b[j], acc[i][j0 + j]);
        };
#pragma unroll
        for (int i = 0; i < 2; ++i) wa0[i] = frag8_at(0, true, i);
#pragma unroll
        for (int j = 0; j < 2; ++j) xb[j] = frag8_at(0, false, j);
        for (int p = 0; p < np; ++p) {
            const int s0 = 2 * p, s1 = 2 * p + 1;
#pragma unroll
            for (int j = 0; j < 2; ++j) xn[j] = frag8_at(s0, false, 2 + j);
            mfmas(wa0, xb, 0);
#pragma unroll
            for (int i = 0; i < 2; ++i) wa1[i] = frag8_at(s1, true, i);
#pragma unroll
            for (int j = 0; j < 2; ++j) xb[j] = frag8_at(s1, false, j);
            mfmas(wa0, xn, 2);
#pragma unroll
            for (int j = 0; j < 2; ++j) xn[j] = frag8_at(s1, false, 2 + j);
            mfmas(wa1, xb, 0);
            meet(p);
#pragma unroll
            for (int i = 0; i < 2; ++i) wa0[i] = frag8_at(s1 + 1, true, i);
#pragma unroll
            for (int j = 0; j < 2; ++j) xb[j] = frag8_at(s1 + 1, false, j);
            mfmas(wa1, xn, 2);
        }
    }
    __builtin_amdgcn_s_setprio(0);

    // Epilogue: the 4-wave tile's, on the wave's 128 x 64 (block (i, j): lane holds out[m][n]
    // for m = j-block row l%32, n = i-block column 8·(r/4) + 4·(l/32) + r%4).
    fence();
    wait_vmcnt<0>();
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    fence();
    const int nl = n0 + wn * 64 + 4 * fq;
    float4 wsv[2][4];
    uint2 bv[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int c = nl - n0 + i * 32 + 8 * g;
            wsv[i][g] = *reinterpret_cast<const float4*>(lds + kWsOff8 + 4 * c);
            if constexpr (kBias) bv[i][g] = *reinterpret_cast<const uint2*>(lds + kBiasOff8 + 2 * c);
        }
    float xsv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xsv[j] = *reinterpret_cast<const float*>(lds + kXsOff8 + 4 * (wm * 128 + j * 32 + fr));
    uint8_t* stage = lds + wave * kStageBytes8;
    const int cl = (lane & 7) * 8;  // first of the lane's 8 columns in a stored row
    const int n = n0 + wn * 64 + cl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ml = j * 32 + fr;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float w4[4] = {wsv[i][g].x, wsv[i][g].y, wsv[i][g].z, wsv[i][g].w};
                const uint2 b2 = kBias ? bv[i][g] : make_uint2(0, 0);
                float v[4];
                uint2 packed;
                if constexpr (kKind == kInt8) {
                    // internal/int8_linear.py:445-448: (acc·xs)·ws, each product rounded to float32.
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        v[r] = __fmul_rn(__fmul_rn(static_cast<float>(acc[i][j][4 * g + r]), xsv[j]), w4[r]);
                    packed = make_uint2(finish2<kOutHalf, kBias, kEpi>(v[0], v[1], b2.x),
                                        finish2<kOutHalf, kBias, kEpi>(v[2], v[3], b2.y));
                } else {
                    // internal/fp8_linear.py:92-111: (acc·xs)·ws + bias in float32, one rounding.
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[r] = __fmul_rn(__fmul_rn(acc[i][j][4 * g + r], xsv[j]), w4[r]);
                    if constexpr (kBias) {
                        v[0] = __fadd_rn(v[0], low_of<kOutHalf>(b2.x));
                        v[1] = __fadd_rn(v[1], high_of<kOutHalf>(b2.x));
                        v[2] = __fadd_rn(v[2], low_of<kOutHalf>(b2.y));
                        v[3] = __fadd_rn(v[3], high_of<kOutHalf>(b2.y));
                    }
                    packed = make_uint2(finish2_float<kOutHalf, kEpi>(v[0], v[1]), finish2_float<kOutHalf, kEpi>(v[2], v[3]));
                }
                *reinterpret_cast<uint2*>(stage + ml * kStageRow8 + 2 * (i * 32 + 8 * g + 4 * fq)) = packed;
            }
        wait_lgkmcnt0();  // a wave reads back only its own rows
        // Whole rows: 8 lanes cover one row's 128 bytes, 8 rows an instruction.
#pragma unroll
        for (int r0 = 0; r0 < 32; r0 += 8) {
            const int rl = j * 32 + r0 + (lane >> 3);
            const int m = m0 + wm * 128 + rl;
            const uint4 v = *reinterpret_cast<const uint4*>(stage + rl * kStageRow8 + 2 * cl);
            if (m < M && n < N) *reinterpret_cast<uint4*>(out + static_cast<int64_t>(m) * ldo + n) = v;
        }
    }
}

template <int kKind, bool kOutHalf, bool kBias, int kEpi>
__global__ __launch_bounds__(kThreads8, 1) void gemm8_kernel(
    const uint8_t* __restrict__ X, const uint8_t* __restrict__ W, const float* __restrict__ xs,
    const float* __restrict__ ws, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out,
    int64_t ldo, int M, int N, int K, int tiles_m, int tiles_n) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kLdsBytes8];
    const int2 t = launch_tile(blockIdx.x, tiles_m, tiles_n);
    gemm_tile8<kKind, kOutHalf, kBias, kEpi>(lds, X, W, xs, ws, bias, out, ldo, M, N, K, t.x, t.y);
}

}  // namespace
}  // namespace cozyq
