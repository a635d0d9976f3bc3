// SVDQuant W4A4, int4-g64 variant, on gfx950.
//
// Activation side (one kernel): xs = bf16(x·p); per 64-group of a row s = fp16(amax|xs| / 7),
// code = clamp(rne(xs / s), -8, 7) (0 where s == 0), packed two a byte with element 2k in the low
// nibble; and the low-rank input la = bf16(x · downᵀ), taken from the same registers on the
// 16x16x32 half-precision MFMA (x in its own dtype, down cast to it: internal/svdq_linear.py:
// 598-602).
//
// GEMM: out = Σ_g (Σ_{k∈g} a·w)·sa[m,g]·sw[n,g] + la·upᵀ + bias, one cast. The packed codes are
// unpacked in registers to bytes holding 16·code (a nibble shifted into a byte's top half keeps
// its sign), multiplied on v_mfma_i32_32x32x32_i8 into a fresh int32 partial P per 64-group (two
// MFMAs) that starts from the bits of 1.5·2^23, so it reads as the float 1.5·2^23 + P; one FMA an
// output adds it times sa·sw (an f16 MFMA) into float32 accumulators that start from the
// low-rank product (v_mfma_f32_32x32x16_bf16), and an f32 MFMA takes the 1.5·2^23·sa·sw part out
// again for two groups at a time. The accumulators run in units of 1/256 (the two 16x factors)
// until the epilogue, an exact power of two.
#include "common.h"
#include "kernels.h"

namespace cozyq {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kGroup = 64;
constexpr float kLevels = 7.0f;

// ------------------------------------------------------------------- activation quantize

constexpr int kQRows = 16;  // rows a block (the MFMA's M)
constexpr int kQWaves = 16;  // waves take a row block's 64-groups round-robin

// Eight 16-bit values (one uint4) as float32.
template <bool kHalf>
__device__ __forceinline__ void widen8(const uint4 v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = widen<kHalf>(static_cast<uint16_t>(w[i] & 0xffffu));
        f[2 * i + 1] = widen<kHalf>(static_cast<uint16_t>(w[i] >> 16));
    }
}

// bf16 bits (one uint4) -> fp16 by way of float32, round to nearest even (torch's cast).
__device__ __forceinline__ f16x8 bf16_to_half8(const uint4 v) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    f16x8 h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[2 * i] = static_cast<_Float16>(float_of(w[i] << 16));
        h[2 * i + 1] = static_cast<_Float16>(float_of(w[i] & 0xffff0000u));
    }
    return h;
}

// Block: kQRows rows. Lane l of a wave holds row l%16 and, in each of its groups, the 16
// columns [16·(l/16), +16): the group's amax is two shuffles away, and the same 16 values feed
// two 16x16x32 MFMAs (columns +0..7 and +8..15; down is read with the same pattern, so every
// k is paired with its own down element).
template <bool kHalf, int kR, bool kPl>
__global__ __launch_bounds__(kQWaves * 64) void svdq_quantize_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ p, const uint16_t* __restrict__ down,
    uint8_t* __restrict__ act, uint16_t* __restrict__ ascales, uint16_t* __restrict__ la, int M,
    int K) {
    constexpr int kJ = kR / 16;
    __shared__ float red[kQWaves][kQRows][kR];
    extern __shared__ __attribute__((aligned(16))) float pl[];  // the smoothing factors p[K]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r16 = lane & 15, part = lane >> 4;
    const int m0 = blockIdx.x * kQRows;
    const int m = m0 + r16;
    const int row = m < M ? m : M - 1;  // rows past M read the last row; nothing of theirs is stored
    const int groups = K / kGroup;
    const uint16_t* xrow = x + static_cast<int64_t>(row) * K;

    f32x4 acc[kJ];
#pragma unroll
    for (int j = 0; j < kJ; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // kPl: p once per block into LDS (the block's 16 rows share it; read from memory, every lane
    // fetches its 16 columns' factors itself, 16 times the bytes: C4's shape 14.7 -> 13.7 us).
    if constexpr (kPl) {
        for (int i = 4 * tid; i < K; i += 4 * kQWaves * 64)
            *reinterpret_cast<float4*>(pl + i) = *reinterpret_cast<const float4*>(p + i);
        __syncthreads();
    }
    const float* const pv_src = kPl ? pl : p;

    for (int g = wave; g < groups; g += kQWaves) {
        const int col = kGroup * g + 16 * part;
        const uint4 xa = *reinterpret_cast<const uint4*>(xrow + col);
        const uint4 xb = *reinterpret_cast<const uint4*>(xrow + col + 8);
        uint4 da[kJ], db[kJ];
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
            const uint16_t* drow = down + static_cast<int64_t>(16 * j + r16) * K + col;
            da[j] = *reinterpret_cast<const uint4*>(drow);
            db[j] = *reinterpret_cast<const uint4*>(drow + 8);
        }
        float pv[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 q4 = *reinterpret_cast<const float4*>(pv_src + col + 4 * i);
            pv[4 * i] = q4.x; pv[4 * i + 1] = q4.y; pv[4 * i + 2] = q4.z; pv[4 * i + 3] = q4.w;
        }

        // internal/svdq_linear.py:592-595: bf16(x·p) in float32.
        float v[16];
        widen8<kHalf>(xa, v);
        widen8<kHalf>(xb, v + 8);
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            v[i] = float_of(static_cast<uint32_t>(bf16_rn(v[i] * pv[i])) << 16);
            amax = fmaxf(amax, fabsf(v[i]));
        }
        amax = fmaxf(amax, __shfl_xor(amax, 16));
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        const _Float16 s16 = static_cast<_Float16>(amax / kLevels);
        const float s = static_cast<float>(s16);
        // A zero scale gives code 0 (the law's `where`), and so does an infinite one (v / inf).
        const bool coded = s != 0.0f && s < __builtin_huge_valf();
        const float rs = 1.0f / s;
        uint32_t packed[2] = {0u, 0u};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float c = 0.0f;
            if (coded) c = fminf(fmaxf(__builtin_rintf(div_rn(v[i], s, rs)), -8.0f), 7.0f);
            const uint32_t nib = static_cast<uint32_t>(static_cast<int>(c)) & 0xfu;
            packed[i >> 3] |= nib << (4 * (i & 7));
        }
        if (m < M) {
            const int64_t base = static_cast<int64_t>(m) * (K / 2) + 32 * g + 8 * part;
            *reinterpret_cast<uint2*>(act + base) = make_uint2(packed[0], packed[1]);
            if (part == 0) ascales[static_cast<int64_t>(m) * groups + g] = __builtin_bit_cast(uint16_t, s16);
        }

        // The low-rank input: x (not xs) against down, in x's dtype.
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
            if constexpr (kHalf) {
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(f16x8, xa), bf16_to_half8(da[j]), acc[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(f16x8, xb), bf16_to_half8(db[j]), acc[j], 0, 0, 0);
            } else {
                acc[j] = mfma_bf16(__builtin_bit_cast(bf16x8, xa), __builtin_bit_cast(bf16x8, da[j]), acc[j]);
                acc[j] = mfma_bf16(__builtin_bit_cast(bf16x8, xb), __builtin_bit_cast(bf16x8, db[j]), acc[j]);
            }
        }
    }

    // acc[j]: lane holds rank 16j + l%16 of rows 4·(l/16) + r. Sum the waves' partials.
#pragma unroll
    for (int j = 0; j < kJ; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][4 * part + r][16 * j + r16] = acc[j][r];
    __syncthreads();
    for (int t = tid; t < kQRows * kR; t += kQWaves * 64) {
        const int rl = t / kR, rank = t % kR;
        if (m0 + rl >= M) continue;
        float sum = red[0][rl][rank];
#pragma unroll
        for (int w = 1; w < kQWaves; ++w) sum += red[w][rl][rank];
        la[static_cast<int64_t>(m0 + rl) * kR + rank] = bf16_rn(sum);
    }
}

constexpr int kPlMaxK = 12288;  // widest rows whose p the quantize kernel stages in LDS (48 KB)

template <bool kHalf, int kR>
hipError_t launch_quantize(const void* x, const float* p, const void* down, uint8_t* act,
                           uint16_t* ascales, void* la, int M, int K, hipStream_t s) {
    const int blocks = (M + kQRows - 1) / kQRows;
    auto xp = static_cast<const uint16_t*>(x);
    auto dp = static_cast<const uint16_t*>(down);
    auto lp = static_cast<uint16_t*>(la);
    if (K <= kPlMaxK)
        svdq_quantize_kernel<kHalf, kR, true><<<blocks, kQWaves * 64, static_cast<size_t>(K) * 4, s>>>(
            xp, p, dp, act, ascales, lp, M, K);
    else
        svdq_quantize_kernel<kHalf, kR, false><<<blocks, kQWaves * 64, 0, s>>>(xp, p, dp, act, ascales, lp, M, K);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------ GEMM

constexpr int kTile = 128;                          // output tile edge (M and N)
constexpr int kThreads = 256;                       // 4 waves, each a 64x64 quadrant
constexpr int kStageGroups = 4;                     // 64-groups a stage brings in
constexpr int kRowBytes = kStageGroups * 32;        // packed bytes of one tile row a stage: 128
constexpr int kOpBytes = kTile * kRowBytes;         // one operand's stage: 16 KB
constexpr int kScaleBytes = kStageGroups * kTile * 4;  // one operand's scales of a stage: 2 KB
constexpr int kStageBytes = 2 * kOpBytes + 2 * kScaleBytes;
constexpr int kStages = 2;
constexpr uint32_t kOutOfRange = 0x80000000u;       // a buffer offset past num_records reads zeros
constexpr int kGroupM = 4;                          // M-tiles a tile group spans

__device__ __forceinline__ void fence() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ void wait_all() {
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt, expcnt and lgkmcnt all zero
}

// 16-byte chunk c (0..7) of a 128-byte LDS row r sits at chunk c ^ ((r / 2) % 8). A fragment's
// ds_read_b128 is served 16 lanes (16 consecutive rows at one chunk) at a time over 256 bytes of
// banks (measured on MI355X), so those rows need distinct (r % 2, chunk) pairs; c ^ (r % 8) gave
// rows r and r + 8 the same banks (2-way conflicts on every read). The rows arrive by whole-row
// LDS-DMA, 8 lanes a row, which any such permutation keeps conflict-free.
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

// 32 packed codes (16 bytes, element 2k in the low nibble of byte k) -> bytes holding 16·code,
// as the two 16-byte operands of one group's two MFMAs: each dword's low nibbles shifted up,
// then its high nibbles in place. Both operands are unpacked alike, so every k still meets its
// own partner; only the order of the sum within a group changes, and int32 sums are exact.
__device__ __forceinline__ void unpack16(const i32x4 v, i32x4& h0, i32x4& h1) {
    constexpr uint32_t kTop = 0xf0f0f0f0u;
    uint32_t u[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t d = static_cast<uint32_t>(v[i]);
        u[2 * i] = (d << 4) & kTop;
        u[2 * i + 1] = d & kTop;
    }
    h0 = i32x4{static_cast<int32_t>(u[0]), static_cast<int32_t>(u[1]), static_cast<int32_t>(u[2]), static_cast<int32_t>(u[3])};
    h1 = i32x4{static_cast<int32_t>(u[4]), static_cast<int32_t>(u[5]), static_cast<int32_t>(u[6]), static_cast<int32_t>(u[7])};
}

template <bool kOutHalf>
__device__ __forceinline__ uint16_t round_out(float v) {
    if constexpr (kOutHalf) {
        return narrow<true>(v);
    } else {
        return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));  // RNE
    }
}

// kWide (the group count a multiple of 8, the scale arrays 16-byte aligned): a lane brings one
// row's scales of 8 groups (two stages) as one 16-byte load. Otherwise every (group, row) scale
// is its own 2-byte load, whose 64 lanes touch as many cache lines as rows (a row's scales sit
// groups·2 bytes apart): those loads cost as much time as the code loads.
template <bool kOutHalf, bool kBias, int kR, bool kWide>
__global__ __launch_bounds__(kThreads, 2) void svdq_gemm_kernel(
    const uint8_t* __restrict__ act, const uint16_t* __restrict__ ascales,
    const uint8_t* __restrict__ w, const uint16_t* __restrict__ wscales,
    const uint16_t* __restrict__ la, const uint16_t* __restrict__ up,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int M, int N, int K,
    int tiles_m, int tiles_n) {
    // The stages, then the tile's 128 biases (read by the epilogue, which stages each wave's
    // quadrant in the stage area once the loop is done).
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes + 2 * kTile];
    uint8_t* const bias_l = lds + kStages * kStageBytes;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 31, fq = lane >> 5;

    const int tiles = tiles_m * tiles_n;
    int t = blockIdx.x;
    if ((tiles & 7) == 0) t = (t & 7) * (tiles >> 3) + (t >> 3);
    const int group = t / (kGroupM * tiles_n);
    const int gm = min(kGroupM, tiles_m - group * kGroupM);
    const int within = t - group * kGroupM * tiles_n;
    const int tm = group * kGroupM + within % gm, tn = within / gm;
    const int m0 = __builtin_amdgcn_readfirstlane(tm * kTile);
    const int n0 = __builtin_amdgcn_readfirstlane(tn * kTile);

    const int groups = K / kGroup, half = K / 2;
    const int64_t aspan = static_cast<int64_t>(M - m0) * half, wspan = static_cast<int64_t>(N - n0) * half;
    const uint32_t abytes = aspan > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(aspan);
    const uint32_t wbytes = wspan > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(wspan);
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(act + static_cast<int64_t>(m0) * half), 0, abytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(w + static_cast<int64_t>(n0) * half), 0, wbytes, 0x00020000);

    // Load j (0..3) of a wave fills 16-byte LDS chunks [(4j + wave)·64, +64) of an operand's
    // stage: lane l writes chunk i = that + l, i.e. row i/8, physical chunk i%8, so it reads
    // logical chunk (i%8) ^ (row%8) of the row's 128 stage bytes.
    int rowoff[4], chunk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = (4 * j + wave) * 64 + lane;
        const int r = i >> 3;
        chunk[j] = 16 * swz(r, i & 7);
        rowoff[j] = r * half + chunk[j];
    }
    // Scales, in a stage buffer's scale area (2·kScaleBytes after its codes):
    // - kWide: the area of buffer b%2 holds stages 2b and 2b+1 (groups 8b..8b+7) as [operand]
    //   [row][8 fp16], 16 bytes a row; wave w brings operand w/2, rows 64·(w%2) + lane;
    // - otherwise each stage's own area holds its 4 groups by 2-byte LDS-DMA, which writes each
    //   lane's value into a 4-byte slot: scale (group g, row r) of an operand sits in slot
    //   operand·kTile·4 + g·kTile + r. Load q (0..3) of a wave covers operand c/8, group (c/2)%4
    //   and rows 64·(c%2) + lane, c = 4q + wave.
    // Past the matrix's rows or its last group they read as zeros.
    const int64_t asspan = static_cast<int64_t>(M - m0) * groups * 2, wsspan = static_cast<int64_t>(N - n0) * groups * 2;
    const __amdgpu_buffer_rsrc_t asr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(ascales + static_cast<int64_t>(m0) * groups), 0,
        asspan > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(asspan), 0x00020000);
    const __amdgpu_buffer_rsrc_t wsr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(wscales + static_cast<int64_t>(n0) * groups), 0,
        wsspan > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(wsspan), 0x00020000);

#define COZYQ_SVDQ_ISSUE(stage)                                                                     \
    do {                                                                                            \
        uint8_t* buf_ = lds + ((stage) & 1) * kStageBytes;                                          \
        const int k0_ = (stage) * kRowBytes;                                                        \
        _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                             \
            const uint32_t off_ = (k0_ + chunk[j] < half) ? static_cast<uint32_t>(rowoff[j] + k0_) : kOutOfRange; \
            const int base_ = (4 * j + wave) * 1024;                                                \
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (LdsPtr*)(buf_ + base_), 16, off_, 0, 0, 0); \
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (LdsPtr*)(buf_ + kOpBytes + base_), 16, off_, 0, 0, 0); \
        }                                                                                           \
        if constexpr (kWide) {                                                                      \
            if (((stage) & 1) == 0) {                                                               \
                const int b_ = (stage) >> 1, r_ = 64 * (wave & 1) + lane;                             \
                const uint32_t so_ = 8 * b_ < groups ? static_cast<uint32_t>(2 * (r_ * groups + 8 * b_)) : kOutOfRange; \
                uint8_t* dst_ = lds + (b_ & 1) * kStageBytes + 2 * kOpBytes + (wave >> 1) * 2048 + 1024 * (wave & 1); \
                __builtin_amdgcn_raw_ptr_buffer_load_lds((wave >> 1) ? wsr : asr, (LdsPtr*)dst_, 16, so_, 0, 0, 0); \
            }                                                                                       \
        } else {                                                                                    \
            _Pragma("unroll") for (int q = 0; q < 4; ++q) {                                         \
                const int c_ = 4 * q + wave, g_ = (c_ >> 1) & 3, r_ = 64 * (c_ & 1) + lane;           \
                const int gg_ = (stage) * kStageGroups + g_;                                        \
                const uint32_t so_ = gg_ < groups ? static_cast<uint32_t>(2 * (r_ * groups + gg_)) : kOutOfRange; \
                uint8_t* dst_ = buf_ + 2 * kOpBytes + (c_ >> 3) * kScaleBytes + 4 * (g_ * kTile + 64 * (c_ & 1)); \
                __builtin_amdgcn_raw_ptr_buffer_load_lds((c_ >> 3) ? wsr : asr, (LdsPtr*)dst_, 2, so_, 0, 0, 0); \
            }                                                                                       \
        }                                                                                           \
    } while (0)

    // The first stage and the biases are requested before the low-rank product, so their latency
    // runs under it. Biases: two a lane by 4-byte LDS-DMA (N % 8 == 0: no partial dword).
    COZYQ_SVDQ_ISSUE(0);
    if (kBias && wave == 0) {
        const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(bias + n0), 0, static_cast<uint32_t>(2 * (N - n0)), 0x00020000);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(br, (LdsPtr*)bias_l, 4, 4 * lane, 0, 0, 0);
    }

    // Every MFMA takes the weight side as its A operand and the activation side as B, so block
    // (i, j) — activation rows 32i.., weight columns 32j.. of the quadrant — leaves lane l with
    // row m = 32i + l%32 and columns n = 32j + 8·(r/4) + 4·(l/32) + r%4: runs of four
    // consecutive outputs of one row. The accumulators start as the low-rank product la·upᵀ.
    f32x16 facc[2][2];
    {
        bf16x8 lv[2][kR / 16], uv[2][kR / 16];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int m = min(m0 + wm * 64 + 32 * i + fr, M - 1);
            const int n = min(n0 + wn * 64 + 32 * i + fr, N - 1);
#pragma unroll
            for (int kk = 0; kk < kR / 16; ++kk) {
                lv[i][kk] = *reinterpret_cast<const bf16x8*>(la + static_cast<int64_t>(m) * kR + 16 * kk + 8 * fq);
                uv[i][kk] = *reinterpret_cast<const bf16x8*>(up + static_cast<int64_t>(n) * kR + 16 * kk + 8 * fq);
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
#pragma unroll
                for (int r = 0; r < 16; ++r) facc[i][j][r] = 0.0f;
#pragma unroll
                for (int kk = 0; kk < kR / 16; ++kk)
                    facc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(uv[j][kk], lv[i][kk], facc[i][j], 0, 0, 0);
                // The K loop accumulates 256·(Σ q·q)·sa·sw (the codes enter as 16·q bytes), so
                // the accumulators run in units of 1/256 until the epilogue; both scalings are
                // exact.
#pragma unroll
                for (int r = 0; r < 16; ++r) facc[i][j][r] *= 256.0f;
            }
    }

    // Fragment addresses within a stage (32x32x32: lane l supplies row l%32 and 16 bytes of each
    // 32-byte K half; here 16 packed bytes = 32 codes = both halves of one group per lane
    // group l/32).
    int aoff[2][kStageGroups], boff[2][kStageGroups];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int g = 0; g < kStageGroups; ++g) {
            const int ra = wm * 64 + 32 * i + fr, rb = wn * 64 + 32 * i + fr;
            aoff[i][g] = ra * kRowBytes + 16 * swz(ra, 2 * g + fq);
            boff[i][g] = kOpBytes + rb * kRowBytes + 16 * swz(rb, 2 * g + fq);
        }
    // Scale addresses: a lane's row of block i (activation side) and column of block j (weight
    // side) within the stage's fp16 scale rows.
    const int sa_row = wm * 64 + fr;
    const int sw_col = wn * 64 + fr;

// One 32-code K half of a block's int32 partial (weight fragment A, activation fragment B).
#define COZYQ_MMA(W, X, C) __builtin_amdgcn_mfma_i32_32x32x32_i8((W), (X), (C), 0, 0, 0)
// The first K half starts from the bits of kOffset = 1.5·2^23 instead of zero: |P| <= 2^20 (64
// products of 16·code bytes, each at most 2^14 in magnitude), so the int32 result P + 0x4B400000
// is the float kOffset + P exactly and needs no conversion.
// The kOffset part of two groups' products leaves the accumulators as one f32 MFMA with K = 2.
#define COZYQ_OFF_MMA(SW, SA, C) __builtin_amdgcn_mfma_f32_32x32x2f32((SW), (SA), (C), 0, 0, 0)
// The block's scale products sw[n]·sa[m] as one f16 MFMA with K = 1 (every other k is zero):
// each product of two fp16 values is exact in float32, and lands where the block's partial does.
#define COZYQ_T(SW, SA)                                                                             \
    __builtin_amdgcn_mfma_f32_32x32x16_f16((SW), (SA), f32x16{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0}, 0, 0, 0)
// (The empty asm holds the block's accumulators at this point of the program: without it the
// arithmetic, which touches no memory, drifts past the scheduling fences below.)
// (The partial is reinterpreted as a whole vector: clang's bit cast of one element of a vector
// reads element 0 whatever the index.)
#define COZYQ_RESCALE(P, T, I, J)                                                                   \
    do {                                                                                            \
        const f32x16 f_ = __builtin_bit_cast(f32x16, (P));                                          \
        _Pragma("unroll") for (int r_ = 0; r_ < 16; ++r_)                                           \
            facc[I][J][r_] = __builtin_fmaf(f_[r_], (T)[r_], facc[I][J][r_]);                       \
        asm volatile("" : "+v"(facc[I][J]));                                                        \
    } while (0)

    // One group's scale operands: element 0 of lane group 0 holds the row's (column's) scale;
    // lane group 1's bits are masked to zero (no branch).
    const uint32_t keep = fq == 0 ? 0xffffu : 0u;
    // Stage s's scale of group g (0..3) and row r of operand op (0: activation, 1: weight), its
    // fp16 bits in the low half.
    auto scale_bits = [&](int s, int op, int g, int r) -> uint32_t {
        if constexpr (kWide) {
            return *reinterpret_cast<const uint16_t*>(lds + ((s >> 1) & 1) * kStageBytes + 2 * kOpBytes + op * 2048 +
                                                      16 * r + 2 * (4 * (s & 1) + g));
        } else {
            return *reinterpret_cast<const uint32_t*>(lds + (s & 1) * kStageBytes + 2 * kOpBytes + op * kScaleBytes +
                                                      4 * (g * kTile + r)) & 0xffffu;
        }
    };
    auto frag_of = [](uint32_t bits) { return __builtin_bit_cast(f16x8, i32x4{static_cast<int32_t>(bits), 0, 0, 0}); };
    auto scale_frag = [&](int s, int op, int g, int r) { return frag_of(scale_bits(s, op, g, r) & keep); };

    // A group adds (kOffset + P)·sa·sw per output (one FMA); the kOffset part of a stage's groups
    // 2p and 2p + 1 is taken out by one f32 MFMA with K = 2 a block: lane group l/32 supplies
    // group 2p + l/32's -kOffset·sw[n] (A) and sa[m] (B). Each product is exact in float32
    // (kOffset·sw has 13 significant bits, sa 11), so only the accumulator's rounding enters,
    // at the magnitude of kOffset·sa·sw (2^-24 of it a step).
    constexpr float kOffset = 12582912.0f;  // 1.5·2^23; its bits are 0x4B400000
    auto half_at = [&](int s, int op, int g, int r) {
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(scale_bits(s, op, g, r))));
    };

    const int nstages = (groups + kStageGroups - 1) / kStageGroups;
    constexpr int32_t kBits = 0x4B400000;
    const i32x16 seed = i32x16{kBits, kBits, kBits, kBits, kBits, kBits, kBits, kBits,  // kOffset's bits
                               kBits, kBits, kBits, kBits, kBits, kBits, kBits, kBits};
    fence();
    wait_all();
    __syncthreads();

    // The loop is a pipeline over block steps (4 a group: blocks (0,0), (0,1), (1,0), (1,1) of
    // activation block i and weight block j). Step t issues block t's MFMAs (at even groups first
    // its share of the offset) and rescales block t - 1, whose results arrived meanwhile; each
    // MFMA is followed by a few of the rescale's FMAs in the issue order, so one wave keeps the
    // matrix core and the VALU busy together. The next group's fragments are read from LDS at
    // its first step and unpacked into the registers its blocks free: a[0] after step 1, b[0]
    // after step 2, a[1] and b[1] after step 3.
    i32x16 pp = seed;  // the block in flight: kOffset + P as int32 bits
    f32x16 tp = {};    // its scale products
    i32x4 a[2][2], b[2][2];  // [block][K half], unpacked 16·code bytes of the current group
    f16x8 fa[2], fb[2];      // its scale operands
    // One block step: MFMAs of block (I, J) of group G interleaved with the rescale of the
    // block before it (PI, PJ), when there is one.
#define COZYQ_STEP(G, I, J, PI, PJ, RESCALE_PREV)                                                   \
    do {                                                                                            \
        if constexpr (((G) & 1) == 0)                                                               \
            facc[I][J] = COZYQ_OFF_MMA(ow[J], oa[I], facc[I][J]);                                   \
        const i32x16 q_ = COZYQ_MMA(b[J][0], a[I][0], seed);                                        \
        const i32x16 p_ = COZYQ_MMA(b[J][1], a[I][1], q_);                                          \
        const f32x16 t_ = COZYQ_T(fb[J], fa[I]);                                                    \
        if (RESCALE_PREV) COZYQ_RESCALE(pp, tp, PI, PJ);                                            \
        pp = p_;                                                                                    \
        tp = t_;                                                                                    \
        if constexpr (((G) & 1) == 0) {                                                             \
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                      \
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);                                      \
        }                                                                                           \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  /* MFMA */                              \
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  /* VALU */                              \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                          \
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);                                          \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                          \
        __builtin_amdgcn_sched_group_barrier(0x002, 30, 0);                                         \
        __builtin_amdgcn_sched_barrier(0);                                                          \
    } while (0)

    for (int s = 0; s < nstages; ++s) {
        const bool more = s + 1 < nstages;
        if (more) COZYQ_SVDQ_ISSUE(s + 1);
        const uint8_t* buf = lds + (s & 1) * kStageBytes;
        // A stage past the last group holds zero codes and zero scales: it adds nothing.
        // The offset operands of pair p (groups 2p, 2p + 1): -kOffset·sw of column block j and
        // sa of row block i, lane group l/32 holding group 2p + l/32.
        float ow[2], oa[2];
        auto offsets = [&](int p) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                ow[i] = -kOffset * half_at(s, 1, 2 * p + fq, sw_col + 32 * i);
                oa[i] = half_at(s, 0, 2 * p + fq, sa_row + 32 * i);
            }
        };
        offsets(0);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            unpack16(*reinterpret_cast<const i32x4*>(buf + aoff[i][0]), a[i][0], a[i][1]);
            unpack16(*reinterpret_cast<const i32x4*>(buf + boff[i][0]), b[i][0], b[i][1]);
            fa[i] = scale_frag(s, 0, 0, sa_row + 32 * i);
            fb[i] = scale_frag(s, 1, 0, sw_col + 32 * i);
        }
#pragma unroll
        for (int g = 0; g < kStageGroups; ++g) {
            constexpr int kLast = kStageGroups - 1;
            const int gn = g < kLast ? g + 1 : g;
            i32x4 na[2], nb[2];
            uint32_t nfa[2], nfb[2];  // the next group's scale bits
            if (g < kLast) {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    na[i] = *reinterpret_cast<const i32x4*>(buf + aoff[i][gn]);
                    nb[i] = *reinterpret_cast<const i32x4*>(buf + boff[i][gn]);
                    nfa[i] = scale_bits(s, 0, gn, sa_row + 32 * i) & keep;
                    nfb[i] = scale_bits(s, 1, gn, sw_col + 32 * i) & keep;
                }
            }
            if (g == 2) offsets(1);
            switch (g) {  // (g is unrolled: each case is its own code)
                case 0: COZYQ_STEP(0, 0, 0, 1, 1, s > 0); break;
                case 1: COZYQ_STEP(1, 0, 0, 1, 1, true); break;
                case 2: COZYQ_STEP(2, 0, 0, 1, 1, true); break;
                default: COZYQ_STEP(3, 0, 0, 1, 1, true); break;
            }
            switch (g) {
                case 0: COZYQ_STEP(0, 0, 1, 0, 0, true); break;
                case 1: COZYQ_STEP(1, 0, 1, 0, 0, true); break;
                case 2: COZYQ_STEP(2, 0, 1, 0, 0, true); break;
                default: COZYQ_STEP(3, 0, 1, 0, 0, true); break;
            }
            switch (g) {
                case 0: COZYQ_STEP(0, 1, 0, 0, 1, true); break;
                case 1: COZYQ_STEP(1, 1, 0, 0, 1, true); break;
                case 2: COZYQ_STEP(2, 1, 0, 0, 1, true); break;
                default: COZYQ_STEP(3, 1, 0, 0, 1, true); break;
            }
            if (g < kLast) unpack16(na[0], a[0][0], a[0][1]);
            switch (g) {
                case 0: COZYQ_STEP(0, 1, 1, 1, 0, true); break;
                case 1: COZYQ_STEP(1, 1, 1, 1, 0, true); break;
                case 2: COZYQ_STEP(2, 1, 1, 1, 0, true); break;
                default: COZYQ_STEP(3, 1, 1, 1, 0, true); break;
            }
            if (g < kLast) {
                unpack16(nb[0], b[0][0], b[0][1]);
                unpack16(na[1], a[1][0], a[1][1]);
                unpack16(nb[1], b[1][0], b[1][1]);
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    fa[i] = frag_of(nfa[i]);
                    fb[i] = frag_of(nfb[i]);
                }
            }
        }
        fence();
        wait_all();
        __syncthreads();
    }
    COZYQ_RESCALE(pp, tp, 1, 1);  // the last block
#undef COZYQ_STEP
#undef COZYQ_SVDQ_ISSUE
#undef COZYQ_MMA
#undef COZYQ_OFF_MMA
#undef COZYQ_T
#undef COZYQ_RESCALE

    // Epilogue: + bias, one cast; each run of four outputs goes to the wave's 64x64 quadrant in
    // LDS as one 8-byte write (the stages are free: every wave has passed the loop's last
    // barrier), and whole 128-byte quadrant rows come back as 16-byte reads and stores.
    constexpr int kStageRow = 64 * 2 + 16;  // one staged row: 64 outputs + pad
    uint8_t* const stage = lds + wave * 64 * kStageRow;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int nl = 32 * j + 8 * g + 4 * fq;  // column within the quadrant
            float b4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (kBias) {
                const uint2 bb = *reinterpret_cast<const uint2*>(bias_l + 2 * (wn * 64 + nl));
                b4[0] = widen<kOutHalf>(static_cast<uint16_t>(bb.x & 0xffff));
                b4[1] = widen<kOutHalf>(static_cast<uint16_t>(bb.x >> 16));
                b4[2] = widen<kOutHalf>(static_cast<uint16_t>(bb.y & 0xffff));
                b4[3] = widen<kOutHalf>(static_cast<uint16_t>(bb.y >> 16));
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                uint16_t h[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = facc[i][j][4 * g + e] * 0.00390625f;  // out of the 1/256 units (exact)
                    if constexpr (kBias) v += b4[e];
                    h[e] = round_out<kOutHalf>(v);
                }
                *reinterpret_cast<uint2*>(stage + (32 * i + fr) * kStageRow + 2 * nl) =
                    make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16));
            }
        }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): a wave reads back only its own rows
    const int c = lane & 7;
    const int n = n0 + wn * 64 + 8 * c;  // N % 8 == 0: a chunk is wholly in or out
#pragma unroll
    for (int t8 = 0; t8 < 8; ++t8) {
        const int rl = (lane >> 3) + 8 * t8;
        const int m = m0 + wm * 64 + rl;
        const uint4 v = *reinterpret_cast<const uint4*>(stage + rl * kStageRow + 16 * c);
        if (m < M && n < N) *reinterpret_cast<uint4*>(out + static_cast<int64_t>(m) * N + n) = v;
    }
}

template <bool kOutHalf, bool kBias, int kR>
hipError_t launch_gemm(const uint8_t* act, const uint16_t* ascales, const uint8_t* w,
                       const uint16_t* wscales, const void* la, const void* up, const void* bias,
                       void* out, int M, int N, int K, hipStream_t s) {
    const int tiles_m = (M + kTile - 1) / kTile, tiles_n = (N + kTile - 1) / kTile;
    const bool wide = (K / kGroup) % 8 == 0 && reinterpret_cast<uintptr_t>(ascales) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(wscales) % 16 == 0;
    auto kernel = wide ? svdq_gemm_kernel<kOutHalf, kBias, kR, true> : svdq_gemm_kernel<kOutHalf, kBias, kR, false>;
    kernel<<<tiles_m * tiles_n, kThreads, 0, s>>>(
        act, ascales, w, wscales, static_cast<const uint16_t*>(la),
        static_cast<const uint16_t*>(up), static_cast<const uint16_t*>(bias),
        static_cast<uint16_t*>(out), M, N, K, tiles_m, tiles_n);
    return hipGetLastError();
}

template <int kR>
hipError_t gemm_rank(const uint8_t* act, const uint16_t* ascales, const uint8_t* w,
                     const uint16_t* wscales, const void* la, const void* up, const void* bias,
                     void* out, bool out_half, int M, int N, int K, hipStream_t s) {
    const bool b = bias != nullptr;
    if (out_half)
        return b ? launch_gemm<true, true, kR>(act, ascales, w, wscales, la, up, bias, out, M, N, K, s)
                 : launch_gemm<true, false, kR>(act, ascales, w, wscales, la, up, bias, out, M, N, K, s);
    return b ? launch_gemm<false, true, kR>(act, ascales, w, wscales, la, up, bias, out, M, N, K, s)
             : launch_gemm<false, false, kR>(act, ascales, w, wscales, la, up, bias, out, M, N, K, s);
}

}  // namespace

hipError_t svdq_int4_quantize(const void* x, bool x_half, const float* p, const void* down,
                              uint8_t* act, uint16_t* ascales, void* la, int M, int K, int R,
                              hipStream_t s) {
#define COZYQ_Q(H, RR) \
    if (x_half == H && R == RR) return launch_quantize<H, RR>(x, p, down, act, ascales, la, M, K, s);
    COZYQ_Q(false, 16) COZYQ_Q(false, 32) COZYQ_Q(false, 64)
    COZYQ_Q(true, 16) COZYQ_Q(true, 32) COZYQ_Q(true, 64)
#undef COZYQ_Q
    return hipErrorInvalidValue;
}

hipError_t svdq_int4_gemm(const uint8_t* act, const uint16_t* ascales, const uint8_t* w,
                          const uint16_t* wscales, const void* la, const void* up,
                          const void* bias, void* out, bool out_half, int M, int N, int K, int R,
                          hipStream_t s) {
    if (R == 16) return gemm_rank<16>(act, ascales, w, wscales, la, up, bias, out, out_half, M, N, K, s);
    if (R == 32) return gemm_rank<32>(act, ascales, w, wscales, la, up, bias, out, out_half, M, N, K, s);
    if (R == 64) return gemm_rank<64>(act, ascales, w, wscales, la, up, bias, out, out_half, M, N, K, s);
    return hipErrorInvalidValue;
}

}  // namespace cozyq
