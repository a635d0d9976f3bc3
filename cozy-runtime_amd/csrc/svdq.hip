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
// its sign), multiplied on v_mfma_i32_32x32x32_i8 into a fresh int32 partial per 64-group (two
// MFMAs), and each partial is rescaled into float32 accumulators that start from the low-rank
// product (v_mfma_f32_32x32x16_bf16). The 1/256 of the two 16x factors rides on the activation
// scale, an exact power of two.
#include "common.h"
#include "kernels.h"

namespace cozyq {
namespace {

typedef __attribute__((address_space(3))) void LdsPtr;
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
template <bool kHalf, int kR>
__global__ __launch_bounds__(kQWaves * 64) void svdq_quantize_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ p, const uint16_t* __restrict__ down,
    uint8_t* __restrict__ act, uint16_t* __restrict__ ascales, uint16_t* __restrict__ la, int M,
    int K) {
    constexpr int kJ = kR / 16;
    __shared__ float red[kQWaves][kQRows][kR];

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
            const float4 q4 = *reinterpret_cast<const float4*>(p + col + 4 * i);
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

template <bool kHalf, int kR>
hipError_t launch_quantize(const void* x, const float* p, const void* down, uint8_t* act,
                           uint16_t* ascales, void* la, int M, int K, hipStream_t s) {
    const int blocks = (M + kQRows - 1) / kQRows;
    svdq_quantize_kernel<kHalf, kR><<<blocks, kQWaves * 64, 0, s>>>(
        static_cast<const uint16_t*>(x), p, static_cast<const uint16_t*>(down), act, ascales,
        static_cast<uint16_t*>(la), M, K);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------ GEMM

constexpr int kTile = 128;                          // output tile edge (M and N)
constexpr int kThreads = 256;                       // 4 waves, each a 64x64 quadrant
constexpr int kStageGroups = 4;                     // 64-groups a stage brings in
constexpr int kRowBytes = kStageGroups * 32;        // packed bytes of one tile row a stage: 128
constexpr int kOpBytes = kTile * kRowBytes;         // one operand's stage: 16 KB
constexpr int kScaleBytes = kStageGroups * kTile * 2;  // fp16 scales [group][row]: 1 KB
constexpr int kStageBytes = 2 * kOpBytes + 2 * kScaleBytes;
constexpr int kStages = 2;
constexpr uint32_t kOutOfRange = 0x80000000u;       // a buffer offset past num_records reads zeros
constexpr int kGroupM = 4;                          // M-tiles a tile group spans

__device__ __forceinline__ void fence() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ void wait_all() {
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt, expcnt and lgkmcnt all zero
}

// 16-byte chunk c (0..7) of a 128-byte LDS row r sits at chunk c ^ (r % 8): 8 consecutive rows
// read at one chunk hit 8 distinct 16-byte bank groups.
__device__ __forceinline__ int swz(int r, int c) { return c ^ (r & 7); }

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

template <bool kOutHalf, bool kBias, int kR>
__global__ __launch_bounds__(kThreads, 2) void svdq_gemm_kernel(
    const uint8_t* __restrict__ act, const uint16_t* __restrict__ ascales,
    const uint8_t* __restrict__ w, const uint16_t* __restrict__ wscales,
    const uint16_t* __restrict__ la, const uint16_t* __restrict__ up,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int M, int N, int K,
    int tiles_m, int tiles_n) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes];

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
    // The stage's scales: threads 0..127 the activation rows, 128..255 the weight rows; one
    // row's kStageGroups fp16 scales each, zero past the matrix.
    const bool wside = tid >= kTile;
    const int srow = tid & (kTile - 1);
    const int sglobal = (wside ? n0 : m0) + srow;
    const bool srow_ok = sglobal < (wside ? N : M);
    const uint16_t* sbase = (wside ? wscales : ascales) + static_cast<int64_t>(srow_ok ? sglobal : 0) * groups;

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
    } while (0)

    auto load_scales = [&](int stage, uint16_t* sv) {
#pragma unroll
        for (int g = 0; g < kStageGroups; ++g) {
            const int gg = stage * kStageGroups + g;
            sv[g] = (srow_ok && gg < groups) ? sbase[gg] : static_cast<uint16_t>(0);
        }
    };
    auto store_scales = [&](int stage, const uint16_t* sv) {
        uint16_t* dst = reinterpret_cast<uint16_t*>(lds + (stage & 1) * kStageBytes + 2 * kOpBytes +
                                                    (wside ? kScaleBytes : 0));
#pragma unroll
        for (int g = 0; g < kStageGroups; ++g) dst[g * kTile + srow] = sv[g];
    };

    // Accumulators start as the low-rank product la·upᵀ. Block (i, j) of the quadrant: lane l
    // holds column n = j-block + l%32 and rows m = i-block + 8·(r/4) + 4·(l/32) + r%4.
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
                    facc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lv[i][kk], uv[j][kk], facc[i][j], 0, 0, 0);
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

// One group's int32 partial of a 32x32 block: two MFMAs over its two 32-code K halves.
#define COZYQ_MMA(A, B)                                                                             \
    __builtin_amdgcn_mfma_i32_32x32x32_i8((A)[1], (B)[1],                                          \
        __builtin_amdgcn_mfma_i32_32x32x32_i8((A)[0], (B)[0], i32x16{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0}, 0, 0, 0), 0, 0, 0)
// The block's scale products sa[m]·sw[n] as one f16 MFMA with K = 1 (every other k is zero):
// each product of two fp16 values is exact in float32, and lands where the block's partial does.
#define COZYQ_T(SA, SB)                                                                             \
    __builtin_amdgcn_mfma_f32_32x32x16_f16((SA), (SB), f32x16{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0}, 0, 0, 0)
// (The empty asm holds the block's accumulators at this point of the program: without it the
// arithmetic, which touches no memory, drifts past the scheduling fences below.)
#define COZYQ_RESCALE(P, T, I, J)                                                                   \
    do {                                                                                            \
        _Pragma("unroll") for (int r_ = 0; r_ < 16; ++r_)                                           \
            facc[I][J][r_] = __builtin_fmaf(static_cast<float>((P)[r_]), (T)[r_], facc[I][J][r_]); \
        asm volatile("" : "+v"(facc[I][J]));                                                        \
    } while (0)

    // One group's scale operands: element 0 of lane group 0 holds the row's (column's) scale;
    // lane group 1's bits are masked to zero (no branch).
    const uint32_t keep = fq == 0 ? 0xffffu : 0u;
    auto scale_frag = [&](const uint16_t* base, int idx) {
        const uint32_t bits = static_cast<uint32_t>(base[idx]) & keep;
        return __builtin_bit_cast(f16x8, i32x4{static_cast<int32_t>(bits), 0, 0, 0});
    };

    const int nstages = (groups + kStageGroups - 1) / kStageGroups;
    uint16_t sv[kStageGroups];
    COZYQ_SVDQ_ISSUE(0);
    load_scales(0, sv);
    store_scales(0, sv);
    fence();
    wait_all();
    __syncthreads();

    for (int s = 0; s < nstages; ++s) {
        const bool more = s + 1 < nstages;
        if (more) {
            COZYQ_SVDQ_ISSUE(s + 1);
            load_scales(s + 1, sv);
        }
        const uint8_t* buf = lds + (s & 1) * kStageBytes;
        const uint16_t* sa_l = reinterpret_cast<const uint16_t*>(buf + 2 * kOpBytes);
        const uint16_t* sw_l = reinterpret_cast<const uint16_t*>(buf + 2 * kOpBytes + kScaleBytes);
        // A stage past the last group holds zero codes and zero scales: it adds nothing.
        //
        // Each group runs as four segments that the scheduler may not reorder across: a
        // segment issues the next block's partial and scale-product MFMAs and then rescales the
        // block before it (one conversion and one FMA an output), so the matrix core works
        // while the vector unit rescales. The next group's fragments are read from LDS two or
        // three segments before their use.
        i32x4 a[2][2], b[2][2];  // [block][K half], unpacked 16·code bytes
        {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                unpack16(*reinterpret_cast<const i32x4*>(buf + aoff[i][0]), a[i][0], a[i][1]);
                unpack16(*reinterpret_cast<const i32x4*>(buf + boff[i][0]), b[i][0], b[i][1]);
            }
        }
#pragma unroll
        for (int g = 0; g < kStageGroups; ++g) {
            constexpr int kLast = kStageGroups - 1;
            i32x4 na[2], nb[2];
            const f16x8 fa0 = scale_frag(sa_l, g * kTile + sa_row), fa1 = scale_frag(sa_l, g * kTile + sa_row + 32);
            const f16x8 fb0 = scale_frag(sw_l, g * kTile + sw_col), fb1 = scale_frag(sw_l, g * kTile + sw_col + 32);
            // Segment A: blocks (0,0) and (0,1) issued; next fragments requested; (0,0) rescaled.
            const i32x16 p00 = COZYQ_MMA(a[0], b[0]);
            const f32x16 t00 = COZYQ_T(fa0, fb0);
            const i32x16 p01 = COZYQ_MMA(a[0], b[1]);
            const f32x16 t01 = COZYQ_T(fa0, fb1);
            if (g < kLast) {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    na[i] = *reinterpret_cast<const i32x4*>(buf + aoff[i][g < kLast ? g + 1 : g]);
                    nb[i] = *reinterpret_cast<const i32x4*>(buf + boff[i][g < kLast ? g + 1 : g]);
                }
            }
            COZYQ_RESCALE(p00, t00, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            // Segment B: block (1,0) issued; (0,1) rescaled.
            const i32x16 p10 = COZYQ_MMA(a[1], b[0]);
            const f32x16 t10 = COZYQ_T(fa1, fb0);
            COZYQ_RESCALE(p01, t01, 0, 1);
            __builtin_amdgcn_sched_barrier(0);
            // Segment C: block (1,1) issued; (1,0) rescaled.
            const i32x16 p11 = COZYQ_MMA(a[1], b[1]);
            const f32x16 t11 = COZYQ_T(fa1, fb1);
            COZYQ_RESCALE(p10, t10, 1, 0);
            __builtin_amdgcn_sched_barrier(0);
            // Segment D: the next group's fragments unpacked; (1,1) rescaled.
            if (g < kLast) {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    unpack16(na[i], a[i][0], a[i][1]);
                    unpack16(nb[i], b[i][0], b[i][1]);
                }
            }
            COZYQ_RESCALE(p11, t11, 1, 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (more) store_scales(s + 1, sv);
        fence();
        wait_all();
        __syncthreads();
    }
#undef COZYQ_SVDQ_ISSUE
#undef COZYQ_MMA
#undef COZYQ_T
#undef COZYQ_RESCALE

    // Epilogue: + bias, one cast, 2-byte stores (32 consecutive columns a row per instruction).
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + 32 * j + fr;
        float bv = 0.0f;
        if constexpr (kBias) bv = widen<kOutHalf>(bias[min(n, N - 1)]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * fq + (r & 3);
                if (m < M && n < N) {
                    float v = facc[i][j][r] * 0.00390625f;  // out of the 1/256 units (exact)
                    if constexpr (kBias) v += bv;
                    out[static_cast<int64_t>(m) * N + n] = round_out<kOutHalf>(v);
                }
            }
    }
}

template <bool kOutHalf, bool kBias, int kR>
hipError_t launch_gemm(const uint8_t* act, const uint16_t* ascales, const uint8_t* w,
                       const uint16_t* wscales, const void* la, const void* up, const void* bias,
                       void* out, int M, int N, int K, hipStream_t s) {
    const int tiles_m = (M + kTile - 1) / kTile, tiles_n = (N + kTile - 1) / kTile;
    svdq_gemm_kernel<kOutHalf, kBias, kR><<<tiles_m * tiles_n, kThreads, 0, s>>>(
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
