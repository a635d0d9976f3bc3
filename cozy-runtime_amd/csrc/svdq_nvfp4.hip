// SVDQuant W4A4 with nvfp4 operands (svdq.nvfp4) on gfx950: the reference's `svdq_quantize` and
// `svdq_gemm` (kernels/csrc/gemm.cpp:169-190; law internal/svdq_linear.py:582-659), plus the
// activation's second level g_x (`activation_scale`, :582-590), which the reference takes with
// torch ops.
//
// Activation side (one kernel): xs = bf16(x·p); per 16-block of a row the E4M3 scale
// e4m3(clamp(amax|xs| / (6·g), 2^-9, 448)) and each element's E2M1 code by the law's threshold
// count on |xs / (scale·g)| (ties to the even code), sign in bit 3, packed two a byte with element
// 2k in the low nibble: act [Rows(M), K/2] and ascales [Rows(M), K/16] row-major, Rows(M) = M
// rounded up to 256, rows past M zero. The low-rank input la = bf16(x · downᵀ) [Rows(M), R] comes
// from the same registers on the 16x16x32 half-precision MFMA (x in its own dtype, down cast to
// it: :598-602).
//
// GEMM: out = (A·Wᵀ)·g_x·g_w·c[n] + la·upᵀ + bias[n], rounded once. gfx950's FP4 MFMA scales
// blocks of 32 by E8M0 exponents (and v_cvt_scalef32_*_fp4 reads only its scale's exponent), so
// nvfp4's E4M3 scales per 16 cannot ride on it. Instead each operand element is decoded exactly
// into fp16: E2M1 (v_cvt_scalef32_pk_f16_fp4 at scale 1) times its E4M3 scale (v_pk_mul_f16; the
// product has at most 6 significant bits and lies in [2^-10, 2688], so fp16 holds it exactly),
// and the products are summed in float32 on v_mfma_f32_32x32x16_f16. The 256x256 tile, LDS layout
// and fragment schedule are gemm_tile.h's int8 ones: a 128-byte LDS row holds 64 fp16 elements of
// K, which the f16 MFMA consumes 32 bytes a step exactly as the int8 MFMA does. Staging goes
// through registers: each thread loads one A row's and one W row's 32 code bytes and 4 scale
// bytes for a buffer, decodes them one buffer ahead of the MFMAs that read them, and writes the
// fp16 rows into the swizzled buffer. The epilogue scales the accumulators by g_x·g_w·c[n], adds
// la·upᵀ into the same accumulators on v_mfma_f32_32x32x16_bf16, adds the bias and rounds once.
#include "gemm_tile.h"

namespace cozyq {
namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr float kLevelsMax = 448.0f * 6.0f;  // internal/svdq_linear.py:44
constexpr float kBlockFloor = 0x1p-9f;       // internal/svdq_linear.py:46: E4M3's least subnormal
constexpr float kInputFloor = 1e-30f;        // internal/svdq_linear.py:590
constexpr int kPadRows = 256;                // the operand's row padding (the GEMM's row tile)

__host__ __device__ __forceinline__ int padded_rows(int M) { return (M + kPadRows - 1) / kPadRows * kPadRows; }

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

// ------------------------------------------------------------ the activation's second level

__global__ void input_scale_init(uint32_t* g) { *g = bits_of(kInputFloor); }

// g = max(max over x of fl(|x|·p[col]) / 2688, 1e-30). The law takes amax over rows first, then
// · p, then the max: the same value, since fl(a·p) is monotonic in a for p > 0; the division and
// the clamp are monotonic too, so each workgroup's candidate enters by an unsigned max of its
// (non-negative) float bits into *g, which input_scale_init set to the floor. Maxima propagate
// NaN, as torch's amax does, so an x holding a NaN gives g = NaN, as the law does.
// Atomics on the one word serialize (~10 ns each measured on MI355X, against ~6 us for the whole
// read at C4's size), so there are few workgroups, each of many waves: ~256 of kScaleGroups x
// kScaleThreads threads, and a workgroup whose candidate does not exceed what *g already holds
// skips its atomic. Thread (t, q) of workgroup (bx, by) takes the 8-column chunk
// kScaleThreads·bx + t of the runs of kScaleRows rows kScaleRows·(kScaleGroups·by + q), then
// every kScaleGroups·gridDim.y-th run; a run's loads are in flight together (a wave reads a
// 1 KiB piece of each row), rows past M repeat the last.
constexpr int kScaleThreads = 128;
constexpr int kScaleGroups = 4;
constexpr int kScaleRows = 8;

template <bool kHalf>
__global__ __launch_bounds__(kScaleThreads * kScaleGroups) void input_scale_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ p, int M, int K, uint32_t* __restrict__ g) {
    __shared__ float red[kScaleThreads * kScaleGroups / 64];
    const int t = threadIdx.x % kScaleThreads, q = threadIdx.x / kScaleThreads;
    const int c = blockIdx.x * kScaleThreads + t;
    float m = 0.0f;
    if (c < K / 8) {
        float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // max |x| per column over the rows
        for (int r0 = (blockIdx.y * kScaleGroups + q) * kScaleRows; r0 < M;
             r0 += gridDim.y * kScaleGroups * kScaleRows) {
            uint4 v[kScaleRows];
#pragma unroll
            for (int r = 0; r < kScaleRows; ++r)
                v[r] = *reinterpret_cast<const uint4*>(x + static_cast<int64_t>(min(r0 + r, M - 1)) * K + 8 * c);
#pragma unroll
            for (int r = 0; r < kScaleRows; ++r) {
                float f[8];
                widen8<kHalf>(v[r], f);
#pragma unroll
                for (int i = 0; i < 8; ++i) a[i] = nan_max(a[i], fabsf(f[i]));
            }
        }
        const float4 p0 = *reinterpret_cast<const float4*>(p + 8 * c);
        const float4 p1 = *reinterpret_cast<const float4*>(p + 8 * c + 4);
        const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) m = nan_max(m, __fmul_rn(a[i], pv[i]));
    }
    m = wave_max_nan(m);  // every lane of the workgroup active
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < kScaleThreads * kScaleGroups / 64; ++w) m = nan_max(m, red[w]);
        // A NaN anywhere in x makes g NaN, as the law's amax and clamp do; its bits (a positive
        // NaN, |x| cleared the sign) exceed every non-negative float's, so it wins the max.
        const uint32_t bits = bits_of(nan_max(__fdiv_rn(m, kLevelsMax), kInputFloor));
        if (bits > __hip_atomic_load(g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) atomicMax(g, bits);
    }
}

// ------------------------------------------------------------------- activation quantize

constexpr int kQRows = 16;  // rows a block (the MFMA's M)
constexpr int kQGroup = 64;  // columns a wave takes at a time: four 16-blocks, one a lane group

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

// The E2M1 code of a (already |xs / (scale·g)|): the law's threshold count, nearest value with
// ties to the even code (internal/svdq_linear.py:613-616).
__device__ __forceinline__ uint32_t e2m1_count(float a) {
    return static_cast<uint32_t>(a > 0.25f) + static_cast<uint32_t>(a >= 0.75f) +
           static_cast<uint32_t>(a > 1.25f) + static_cast<uint32_t>(a >= 1.75f) +
           static_cast<uint32_t>(a > 2.5f) + static_cast<uint32_t>(a >= 3.5f) +
           static_cast<uint32_t>(a > 5.0f);
}

// xs / (scale·g) for v_cvt_scalef32_pk_fp4_f32 at unit scale. That conversion (nearest, ties to
// the even code, saturating at 6) gives the law's threshold count, sign included, on every finite
// nonzero quotient and on ±inf (held against e2m1_count over all 2^32 float32 bit patterns on
// MI355X; cozyq_probe_e2m1's test repeats it on every float32 of [2^-4, 2^4)); it writes the sign of −0 and converts NaN to 6, where the law writes code 0 for
// xs = −0 and NaN. So −0 becomes +0 first and NaN gives +0. Otherwise the quotient is RN(xs / sg)
// (div_rn, for finite xs and finite sg > 0).
__device__ __forceinline__ float e2m1_quotient(float xs, float sg, float rs) {
    const float z = __fadd_rn(xs, 0.0f);  // −0 → +0, everything else unchanged
    const float q = div_rn(z, sg, rs);
    return z == z ? q : 0.0f;
}

// Codes of quotients a and b into byte kByte of `word` (a in the low nibble).
template <int kByte>
__device__ __forceinline__ uint32_t put_e2m1_pair(uint32_t word, float a, float b) {
    return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, a, b, 1.0f, kByte);
}

template <int kR>
constexpr int quantize_waves() { return kR == 128 ? 8 : 16; }  // the partial sums fit the LDS

// Block: kQRows rows (of Rows(M)). Lane l of a wave holds row l%16 and, in each of its 64-column
// groups, the 16 columns [16·(l/16), +16): exactly one nvfp4 block, so its amax stays in the
// lane, and the same 16 values feed two 16x16x32 MFMAs against down (read with the same
// pattern, so every k meets its own down element).
template <bool kHalf, int kR, bool kPl>
__global__ __launch_bounds__(quantize_waves<kR>() * 64) void nvfp4_quantize_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ p, const float* __restrict__ g,
    const uint16_t* __restrict__ down, uint8_t* __restrict__ act, uint8_t* __restrict__ ascales,
    uint16_t* __restrict__ la, int M, int K) {
    constexpr int kWaves = quantize_waves<kR>();
    constexpr int kJ = kR / 16;
    __shared__ float red[kWaves][kQRows][kR];
    extern __shared__ __attribute__((aligned(16))) float pl[];  // kPl: the smoothing factors p[K]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r16 = lane & 15, part = lane >> 4;
    const int m0 = blockIdx.x * kQRows;
    const int m = m0 + r16;
    const bool live = m < M;  // rows in [M, Rows(M)) are written as zeros
    const int row = live ? m : M - 1;
    const int groups = K / kQGroup;
    const uint16_t* xrow = x + static_cast<int64_t>(row) * K;
    const float gv = g[0];
    const float six_g = __fmul_rn(6.0f, gv);

    f32x4 acc[kJ];
#pragma unroll
    for (int j = 0; j < kJ; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // kPl: p once per block into LDS (the block's rows share it; read from memory, every lane
    // fetches its 16 columns' factors itself, 16 times the bytes).
    if constexpr (kPl) {
        for (int i = 4 * tid; i < K; i += 4 * kWaves * 64)
            *reinterpret_cast<float4*>(pl + i) = *reinterpret_cast<const float4*>(p + i);
        __syncthreads();
    }

    // A group's operands: the lane's 16 elements of its row, their p, and down's rows at the same
    // columns. The next group's are loaded before the current one is worked on, with no branch
    // around the loads (past the wave's last group they load that group again).
    struct Group {
        uint4 xa, xb, da[kJ], db[kJ];
        float4 p4[4];
    };
    auto fetch = [&](int gi, Group& in) {
        const int col = kQGroup * gi + 16 * part;
        in.xa = *reinterpret_cast<const uint4*>(xrow + col);
        in.xb = *reinterpret_cast<const uint4*>(xrow + col + 8);
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
            const uint16_t* drow = down + static_cast<int64_t>(16 * j + r16) * K + col;
            in.da[j] = *reinterpret_cast<const uint4*>(drow);
            in.db[j] = *reinterpret_cast<const uint4*>(drow + 8);
        }
        if constexpr (!kPl) {
#pragma unroll
            for (int i = 0; i < 4; ++i) in.p4[i] = *reinterpret_cast<const float4*>(p + col + 4 * i);
        }
    };
    Group cur, nxt;
    fetch(min(wave, groups - 1), cur);
    for (int gi = wave; gi < groups; gi += kWaves) {
        fetch(min(gi + kWaves, groups - 1), nxt);
        const uint4 xa = cur.xa, xb = cur.xb;
        if constexpr (kPl) {
            const int col = kQGroup * gi + 16 * part;
#pragma unroll
            for (int i = 0; i < 4; ++i) cur.p4[i] = *reinterpret_cast<const float4*>(pl + col + 4 * i);
        }
        const float pv[16] = {cur.p4[0].x, cur.p4[0].y, cur.p4[0].z, cur.p4[0].w, cur.p4[1].x, cur.p4[1].y,
                              cur.p4[1].z, cur.p4[1].w, cur.p4[2].x, cur.p4[2].y, cur.p4[2].z, cur.p4[2].w,
                              cur.p4[3].x, cur.p4[3].y, cur.p4[3].z, cur.p4[3].w};

        // internal/svdq_linear.py:592-595: xs = bf16(x·p), a pair rounded in one
        // v_cvt_pk_bf16_f32 (round to nearest even, as bf16_rn); :609-611 the block scale.
        float v[16];
        widen8<kHalf>(xa, v);
        widen8<kHalf>(xb, v + 8);
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            const uint32_t pr = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                f32x2{__fmul_rn(v[i], pv[i]), __fmul_rn(v[i + 1], pv[i + 1])}, bf16x2));
            v[i] = float_of(pr << 16);
            v[i + 1] = float_of(pr & 0xffff0000u);
            amax = nan_max(amax, nan_max(fabsf(v[i]), fabsf(v[i + 1])));
        }
        // NaN-propagating, as the law's amax and clamp: a block holding a NaN gets the E4M3 NaN
        // scale, and then every code is the threshold count of NaN (0), + 8 where x < 0.
        const float ratio = nan_min(nan_max(__fdiv_rn(amax, six_g), kBlockFloor), kE4m3Max);
        const uint32_t sb = e4m3_rn(ratio);
        const float sg = __fmul_rn(e4m3_value(sb), gv);
        uint32_t packed[2] = {0u, 0u};
        if (amax < __builtin_huge_valf() && sg < __builtin_huge_valf()) {
            // :612-616: the codes, two a conversion (element 2k in the low nibble).
            const float rs = __fdiv_rn(1.0f, sg);
            float q[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) q[i] = e2m1_quotient(v[i], sg, rs);
            packed[0] = put_e2m1_pair<0>(packed[0], q[0], q[1]);
            packed[0] = put_e2m1_pair<1>(packed[0], q[2], q[3]);
            packed[0] = put_e2m1_pair<2>(packed[0], q[4], q[5]);
            packed[0] = put_e2m1_pair<3>(packed[0], q[6], q[7]);
            packed[1] = put_e2m1_pair<0>(packed[1], q[8], q[9]);
            packed[1] = put_e2m1_pair<1>(packed[1], q[10], q[11]);
            packed[1] = put_e2m1_pair<2>(packed[1], q[12], q[13]);
            packed[1] = put_e2m1_pair<3>(packed[1], q[14], q[15]);
        } else {
            // An infinite block maximum or scale: the law's divisions and threshold count as
            // written.
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t code = e2m1_count(fabsf(__fdiv_rn(v[i], sg))) + (v[i] < 0.0f ? 8u : 0u);
                packed[i >> 3] |= code << (4 * (i & 7));
            }
        }
        if (!live) packed[0] = packed[1] = 0u;
        const int64_t base = static_cast<int64_t>(m) * (K / 2) + 32 * gi + 8 * part;
        *reinterpret_cast<uint2*>(act + base) = make_uint2(packed[0], packed[1]);
        ascales[static_cast<int64_t>(m) * (K / 16) + 4 * gi + part] = live ? static_cast<uint8_t>(sb) : 0;

        // The low-rank input: x (not xs) against down, in x's dtype.
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
            if constexpr (kHalf) {
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(f16x8, xa), bf16_to_half8(cur.da[j]), acc[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(f16x8, xb), bf16_to_half8(cur.db[j]), acc[j], 0, 0, 0);
            } else {
                acc[j] = mfma_bf16(__builtin_bit_cast(bf16x8, xa), __builtin_bit_cast(bf16x8, cur.da[j]), acc[j]);
                acc[j] = mfma_bf16(__builtin_bit_cast(bf16x8, xb), __builtin_bit_cast(bf16x8, cur.db[j]), acc[j]);
            }
        }
        cur = nxt;
    }

    // acc[j]: lane holds rank 16j + l%16 of rows 4·(l/16) + r. Sum the waves' partials.
#pragma unroll
    for (int j = 0; j < kJ; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][4 * part + r][16 * j + r16] = acc[j][r];
    __syncthreads();
    for (int t = tid; t < kQRows * kR; t += kWaves * 64) {
        const int rl = t / kR, rank = t % kR;
        float sum = red[0][rl][rank];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) sum += red[w][rl][rank];
        la[static_cast<int64_t>(m0 + rl) * kR + rank] = m0 + rl < M ? bf16_rn(sum) : 0;
    }
}

template <bool kHalf, int kR>
hipError_t launch_quantize(const void* x, const float* p, const float* g, const void* down,
                           uint8_t* act, uint8_t* ascales, void* la, int M, int K, hipStream_t s) {
    const int blocks = padded_rows(M) / kQRows;
    auto xp = static_cast<const uint16_t*>(x);
    auto dp = static_cast<const uint16_t*>(down);
    auto lp = static_cast<uint16_t*>(la);
    // p staged in LDS up to 12288 columns (48 KB beside the partial sums).
    if (K <= 12288)
        nvfp4_quantize_kernel<kHalf, kR, true><<<blocks, quantize_waves<kR>() * 64, static_cast<size_t>(K) * 4, s>>>(
            xp, p, g, dp, act, ascales, lp, M, K);
    else
        nvfp4_quantize_kernel<kHalf, kR, false><<<blocks, quantize_waves<kR>() * 64, 0, s>>>(
            xp, p, g, dp, act, ascales, lp, M, K);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------ GEMM

// A buffer row's four E4M3 block scales (one byte each, block b = elements 16b..16b+15) as fp16
// pairs (exact: E4M3's range and precision sit inside fp16's), converted at unit scale.
struct RowScales {
    f16x2 lo, hi;  // blocks 0, 1 and 2, 3
};

__device__ __forceinline__ RowScales row_scales(uint32_t sb) {
    return RowScales{__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(sb, 1.0f, false),
                     __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(sb, 1.0f, true)};
}

// The LDS byte address of a pointer into this workgroup's LDS.
__device__ __forceinline__ uint32_t lds_address(const uint8_t* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t*)p));
}

// 16 bytes into LDS by a write the compiler does not count. It waits for every LDS-DMA in flight
// (vmcnt 0) before an LDS write it cannot tell apart from their targets; the W4A16 GEMM writes
// its decoded W while x's lines of the next pair are still landing elsewhere. Younger LDS
// operations the compiler does not know of only make its own lgkmcnt waits stricter.
__device__ __forceinline__ void lds_write16(uint8_t* p, uint4 v) {
    asm volatile("ds_write_b128 %0, %1" ::"v"(lds_address(p)), "v"(__builtin_bit_cast(i32x4, v)) : "memory");
}

// Chunk c (0..7) of a buffer row — elements 8c..8c+7, code dword c, 16-block c/2 — decoded to
// fp16 (E2M1 at unit scale, times the block's scale) and written at its swizzled place in LDS
// row r.
template <bool kUncounted = false>
__device__ __forceinline__ void put_chunk(uint8_t* row, int r, int c, uint32_t dw, const RowScales& s) {
    const _Float16 sc = (c >> 1) == 0 ? s.lo[0] : (c >> 1) == 1 ? s.lo[1] : (c >> 1) == 2 ? s.hi[0] : s.hi[1];
    const f16x2 s2 = {sc, sc};
    const f16x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 1.0f, 0) * s2;
    const f16x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 1.0f, 1) * s2;
    const f16x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 1.0f, 2) * s2;
    const f16x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 1.0f, 3) * s2;
    const uint4 v = make_uint4(__builtin_bit_cast(uint32_t, v0), __builtin_bit_cast(uint32_t, v1),
                               __builtin_bit_cast(uint32_t, v2), __builtin_bit_cast(uint32_t, v3));
    if constexpr (kUncounted)
        lds_write16(row + 16 * swz(r, c), v);
    else
        *reinterpret_cast<uint4*>(row + 16 * swz(r, c)) = v;
}

__device__ __forceinline__ uint32_t dword_of(const uint4& a, const uint4& b, int c) {
    const uint4 v = c < 4 ? a : b;
    const int k = c & 3;
    return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}

// A wave's fill of its W4A16 stage slots by LDS-DMA: each lane's 32 code bytes from `codes` at
// `co` and its scale dword from `scales` at `so`.
__device__ __forceinline__ void fill_stage(uint8_t* st, __amdgpu_buffer_rsrc_t codes, uint32_t co,
                                           __amdgpu_buffer_rsrc_t scales, uint32_t so) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(codes, (LdsPtr*)st, 16, co, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(codes, (LdsPtr*)(st + 1024), 16, co + 16, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(scales, (LdsPtr*)(st + 2048), 4, so, 0, 0, 0);
}

// A lane's slots of a W4A16 stage (its 32 code bytes at 16·lane and 1024 + 16·lane, its scale
// dword at 2048 + 4·lane), read by uncounted LDS reads that complete before it returns.
__device__ __forceinline__ void read_stage(const uint8_t* st, int lane, uint4& lo, uint4& hi, uint32_t& sc) {
    const uint32_t a = lds_address(st);
    i32x4 l, h;
    asm volatile("ds_read_b128 %0, %3\n\t"
                 "ds_read_b128 %1, %3 offset:1024\n\t"
                 "ds_read_b32 %2, %4 offset:2048\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(l), "=&v"(h), "=&v"(sc)
                 : "v"(a + 16 * lane), "v"(a + 4 * lane)
                 : "memory");
    lo = __builtin_bit_cast(uint4, l);
    hi = __builtin_bit_cast(uint4, h);
}

// The W4A16 form's decode into bf16 (x in bf16): E2M1 at unit scale in float32, times the
// block's scale (float32, exact), packed to bf16 (exact: at most 6 significant bits); an
// uncounted write, as the W4A16 GEMM's decode needs.
__device__ __forceinline__ void put_chunk_bf16(uint8_t* row, int r, int c, uint32_t dw, float sc) {
    const int w = static_cast<int>(dw);
    const f32x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
    const f32x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
    const f32x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
    const f32x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
    lds_write16(row + 16 * swz(r, c),
                make_uint4(round2<false>(v0[0] * sc, v0[1] * sc), round2<false>(v1[0] * sc, v1[1] * sc),
                           round2<false>(v2[0] * sc, v2[1] * sc), round2<false>(v3[0] * sc, v3[1] * sc)));
}

template <bool kBf16>
__device__ __forceinline__ f32x16 mfma16x(const i32x8& a, const i32x8& b, int h, f32x16 c) {
    if constexpr (kBf16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, half_of(a, h)),
                                                       __builtin_bit_cast(bf16x8, half_of(b, h)), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, half_of(a, h)),
                                                      __builtin_bit_cast(f16x8, half_of(b, h)), c, 0, 0, 0);
}

// A wave's 8 LDS-DMA loads of one buffer's 16-bit A rows (gemm_tile.h's COZYQ_ISSUE for one
// operand): load j fills the 1 KiB at (4j + wave)·1024 from row offsets rowoff[j] + k0.
__device__ __forceinline__ void issue_lines(__amdgpu_buffer_rsrc_t rsrc, uint8_t* buf, const int (&rowoff)[8],
                                            const int (&chunk)[8], int k0, int row_bytes, int wave) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t off = (k0 + chunk[j] < row_bytes) ? static_cast<uint32_t>(rowoff[j] + k0) : kOutOfRange;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LdsPtr*)(buf + (4 * j + wave) * 1024), 16, off, 0, 0, 0);
    }
}

enum NvMode { kW4A4 = 0, kW4A16 = 1 };
// kW4A16 stages W's codes and scales by LDS-DMA past the tile's buffers, each thread its own
// row: a wave's two 1 KiB code loads and its 256-byte scale load, two stages.
constexpr int kCodeWave = 2 * 1024 + 256, kCodeStage = 4 * kCodeWave;

// One 256x256 output tile per workgroup.
// kW4A4 (svdq.nvfp4): A is the activation's nvfp4 operand (codes + row-major E4M3 scales), both
// operands decoded to fp16; out = (A·Wᵀ)·gx·gw·c + la·upᵀ + bias. c and bias may be null.
// kW4A16 (nvfp4, x 16-bit): A is x itself ([M, K] bf16, or fp16 with kXHalf), brought by LDS-DMA;
// W's E4M3 scales sit in cuBLAS's 128x4 tiles; W is decoded into x's dtype; out = (x·Wᵀ)·gw
// (+ bias). gx, cs, la, up unused.
// kTN (kW4A4): 256 or 192 columns a tile (wide_tile's choice); at 192 each wave owns 128 x 96,
// wave 3 neither loads nor decodes W rows, and every output's sum runs in the same order.
template <int kMode, bool kXHalf, bool kOutHalf, int kTN = 256>
__global__ __launch_bounds__(kThreads, 1) void nvfp4_gemm_kernel(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ As, const uint8_t* __restrict__ W,
    const uint8_t* __restrict__ Ws, const float* __restrict__ gx, const float* __restrict__ gw,
    const float* __restrict__ cs, const uint16_t* __restrict__ la, const uint16_t* __restrict__ up,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int M, int N, int K, int R,
    int tiles_m, int tiles_n) {
    constexpr bool kBf16 = kMode == kW4A16 && !kXHalf;  // the MFMA and W's decoded type
    static_assert(kTN == 256 || (kTN == 192 && kMode == kW4A4), "tile widths: 256, or 192 for W4A4");
    constexpr int kNI = kTN / 64, kHalfN = kTN / 2;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kLdsBytes + (kMode == kW4A16 ? 2 * kCodeStage : 0)];
    const int2 t = launch_tile(blockIdx.x, tiles_m, tiles_n);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = __builtin_amdgcn_readfirstlane(t.x * kTile);
    const int n0 = __builtin_amdgcn_readfirstlane(t.y * kTN);
    const bool wrow = kTN == 256 || wave < 3;  // the wave's threads carry W rows of the tile

    auto rows_view = [&](const void* base, int rows_left, int row_bytes) {
        const int64_t span = static_cast<int64_t>(rows_left) * row_bytes;
        const uint32_t bytes = span > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(span);
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
    };
    const int half_k = K / 2, blocks_k = K / 16;
    const int np = K / 64;  // buffers: 64 elements of K each
    // A: nvfp4 codes and scales (kW4A4) or x's 2K-byte rows (kW4A16).
    const int arow_bytes = kMode == kW4A4 ? half_k : 2 * K;
    const auto ar = rows_view(A + static_cast<int64_t>(m0) * arow_bytes, M - m0, arow_bytes);
    const auto asr = rows_view(As + static_cast<int64_t>(m0) * blocks_k, M - m0, blocks_k);
    const auto wr = rows_view(W + static_cast<int64_t>(n0) * half_k, N - n0, half_k);
    // W's scales: row-major [N, K/16] (kW4A4) or in 128x4 tiles of 512 bytes, K/64 tiles a row of
    // tiles; a row's four block scales of a buffer are one aligned dword of its tile.
    const int col_tiles = K / 64;
    const int64_t tiled_rows = (static_cast<int64_t>(N) + 127) / 128 * 128;
    const auto wsr = kMode == kW4A4
        ? rows_view(Ws + static_cast<int64_t>(n0) * blocks_k, N - n0, blocks_k)
        : rows_view(Ws + static_cast<int64_t>(n0 / 128) * col_tiles * 512,
                    static_cast<int>(tiled_rows - n0), 4 * col_tiles);
    const int n_in = tid;  // the thread's W row within the tile
    const uint32_t tiled_row = static_cast<uint32_t>((n_in >> 7) * col_tiles * 512 + (n_in & 31) * 16 + ((n_in & 127) >> 5) * 4);

    // The epilogue's column operands into LDS ahead of the K loop: c (f32) and the bias (two a
    // lane), for the tile's 256 columns; past N they read as zeros.
    {
        const int cc = 64 * wave + lane;
        if (kMode == kW4A4 && cs != nullptr) {
            const auto cr = rows_view(cs + n0, N - n0, 4);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(cr, (LdsPtr*)(lds + kWsOff + 256 * wave), 4, 4 * cc, 0, 0, 0);
        }
        if (bias != nullptr && wave < 2) {
            const auto br = rows_view(bias + n0, N - n0, 2);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(br, (LdsPtr*)(lds + kBiasOff + 256 * wave), 4, 4 * cc, 0, 0, 0);
        }
    }

    // kW4A16: x's rows by LDS-DMA in whole 128-byte lines, as gemm_tile.h's operands: load j (0..7)
    // of a wave fills rows (4j + wave)·8 + l/8 of the buffer's A half, physical chunk l%8.
    int xrowoff[8], xchunk[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int r = (4 * j + wave) * 8 + (lane >> 3);
        xchunk[j] = 16 * swz(r, lane & 7);
        xrowoff[j] = r * arow_bytes + xchunk[j];
    }
    auto issue_x = [&](int pair) {
        if constexpr (kMode == kW4A16) issue_lines(ar, lds + (pair & 1) * kPairBytes, xrowoff, xchunk, pair * kPairK, arow_bytes, wave);
    };

    // Staging: thread t carries tile row t of W (and of A's codes, kW4A4) for a buffer. kW4A4
    // loads it into registers; kW4A16 into its own slots of stage `pair % 2` past the buffers,
    // two pairs ahead of the decode, and reads it back itself (no barrier: its own loads).
    constexpr bool kDeep = kMode == kW4A16;
    struct Regs {
        uint4 xa0, xa1, wa0, wa1;
        uint32_t xsb, wsb;
    };
    const uint32_t crow = static_cast<uint32_t>(tid * half_k), srow = static_cast<uint32_t>(tid * blocks_k);
    Regs regs{make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), 0u, 0u};
    auto stage_of = [&](int pair) { return lds + kLdsBytes + (pair & 1) * kCodeStage + wave * kCodeWave; };
    // Past the last pair the offsets run past the buffers (zeros) or into later rows: what they
    // bring is decoded into a buffer nothing reads.
    auto load = [&](int pair) {
        const uint32_t co = crow + 32 * pair;
        if constexpr (kDeep) {
            fill_stage(stage_of(pair), wr, co, wsr, tiled_row + 512 * pair);
        } else {
            const uint32_t so = srow + 4 * pair;
            if (wrow) {
                regs.wa0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, co, 0, 0));
                regs.wa1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, co + 16, 0, 0));
                regs.wsb = __builtin_amdgcn_raw_buffer_load_b32(wsr, so, 0, 0);
            }
            regs.xa0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ar, co, 0, 0));
            regs.xa1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ar, co + 16, 0, 0));
            regs.xsb = __builtin_amdgcn_raw_buffer_load_b32(asr, so, 0, 0);
        }
    };
    // The staged rows of `pair` (kW4A16: read back from the thread's slots once its vmcnt wait
    // has seen them land). The reads are written out so that the compiler, which cannot tell the
    // stages apart, does not wait for every LDS-DMA in flight (vmcnt 0) before them; they
    // complete (lgkmcnt 0) before any LDS access the compiler counts.
    auto staged = [&](int pair) {
        if constexpr (kDeep) {
            Regs r = regs;
            read_stage(stage_of(pair), lane, r.wa0, r.wa1, r.wsb);
            return r;
        } else {
            return regs;
        }
    };
    // Slice q (0..15) of the thread's decode of a buffer: kW4A4 the A row's 8 chunks, then W's;
    // kW4A16 one W chunk every other slice.
    struct Scales {
        RowScales x, w;
        float wf[4];
    };
    auto scales_of = [&](const Regs& r) {
        Scales sc;
        sc.x = row_scales(r.xsb);
        sc.w = row_scales(r.wsb);
        if constexpr (kBf16) {
            const f32x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(r.wsb, 1.0f, false);
            const f32x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(r.wsb, 1.0f, true);
            sc.wf[0] = lo[0]; sc.wf[1] = lo[1]; sc.wf[2] = hi[0]; sc.wf[3] = hi[1];
        }
        return sc;
    };
    auto put = [&](uint8_t* buf, int q, const Scales& sc, const Regs& r) {
        if constexpr (kMode == kW4A4) {
            if (q < 8)
                put_chunk(buf + tid * kPairK, tid, q, dword_of(r.xa0, r.xa1, q), sc.x);
            else if (wrow)
                put_chunk(buf + kOpBytes + tid * kPairK, tid, q - 8, dword_of(r.wa0, r.wa1, q - 8), sc.w);
        } else if (q & 1) {
            const int c = q >> 1;
            if constexpr (kBf16)
                put_chunk_bf16(buf + kOpBytes + tid * kPairK, tid, c, dword_of(r.wa0, r.wa1, c), sc.wf[c >> 1]);
            else
                put_chunk<true>(buf + kOpBytes + tid * kPairK, tid, c, dword_of(r.wa0, r.wa1, c), sc.w);
        }
    };
    auto store = [&](int pair, const Regs& r) {
        uint8_t* buf = lds + (pair & 1) * kPairBytes;
        const Scales sc = scales_of(r);
#pragma unroll
        for (int q = 0; q < 16; ++q) put(buf, q, sc, r);
    };

    // Fragment reads as gemm_tile.h's int8 kind: lane l supplies row l%32; lane group l/32 its
    // K chunks; step e of a buffer reads logical chunks 4e + 2h + l/32 (h = 0, 1), each 8 16-bit
    // elements, one MFMA's K half.
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
    };

    f32x16 acc[kNI][4];
#pragma unroll
    for (int i = 0; i < kNI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    auto mfmas = [&](const Frags& c) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < kNI; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x<kBf16>(c.a[i], c.b[j], h, acc[i][j]);
    };
    auto schedule = [&]() {
#pragma unroll
        for (int g = 0; g < 4 * kNI; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // 2 MFMA
        }
        if constexpr (kTN != 256) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    };

    // kW4A4: pair p + 1's register loads are issued after the barrier of step 2p - 1 (pair 1's
    // before the loop) and waited at the top of step 2p, whose slices decode and write them,
    // between that step's MFMAs, into the buffer no wave has read since that barrier; the barrier
    // of step 2p + 1 makes them visible.
    // kW4A16: x's lines of pair p + 2 go by LDS-DMA after the barrier that ends step 2p and must
    // land by the one that ends step 2p + 2; W's rows of pair p + 3 go with them, into the stage
    // that step 2p's decode (of pair p + 1) has just read, and are waited at the top of step
    // 2p + 4. At the top of step 2p a thread's loads in flight are then, in issue order, W(p + 1),
    // x(p + 1), W(p + 2): vmcnt ≤ 11 means W(p + 1) is in, and vmcnt ≤ 3 that x(p + 1) is. Every
    // load is issued, past the last pair too, so those counts hold to the end.
    constexpr int kXIssue = 8, kWIssue = 3;
    // The issue order the counts rely on is pinned by `order()`.
    auto order = [&]() {
        fence();
        __builtin_amdgcn_sched_barrier(0);
    };
    issue_x(0);
    order();
    load(0);
    order();
    if constexpr (kDeep) load(1);
    fence();
    if constexpr (kDeep)
        wait_vmcnt<kWIssue>();
    else
        wait_vmcnt<0>();
    fence();
    store(0, staged(0));
    order();
    issue_x(1);
    order();
    if constexpr (kDeep)
        load(2);
    else if (np > 1)
        load(1);
    fence();
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    fence();

    // Step 2p: 16 slices, each one fragment read for step 2p + 1, two of this step's MFMAs (K
    // half h = q / 8, so that no MFMA waits on the one before it) and one slice of pair p + 1's
    // decode.
    auto even_step = [&](int s, const Frags& cur, Frags& next, const Regs& r) {
        const uint8_t* rbuf = lds + ((s + 1) >> 1 & 1) * kPairBytes;
        const int e = (s + 1) & 1;
        uint8_t* wbuf = lds + (((s >> 1) + 1) & 1) * kPairBytes;
        const Scales sc = scales_of(r);
        i32x4 piece[4][4];  // [i][alo, ahi, blo, bhi]
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int fi = q >> 2, fk = q & 3;
            const int off = fk < 2 ? aoff[e][fk][fi] : boff[e][fk - 2][fi];
            if (fk >= 2 || fi < kNI) piece[fi][fk] = *reinterpret_cast<const i32x4*>(rbuf + off);
            const int h = q >> 3, i = (q >> 1) & 3, j = 2 * (q & 1);
            if (i < kNI) {
                acc[i][j] = mfma16x<kBf16>(cur.a[i], cur.b[j], h, acc[i][j]);
                acc[i][j + 1] = mfma16x<kBf16>(cur.a[i], cur.b[j + 1], h, acc[i][j + 1]);
            }
            put(wbuf, q, sc, r);
            __builtin_amdgcn_sched_barrier(0);  // slices stay in order: decode rides under MFMAs
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i < kNI) next.a[i] = __builtin_shufflevector(piece[i][0], piece[i][1], 0, 1, 2, 3, 4, 5, 6, 7);
            next.b[i] = __builtin_shufflevector(piece[i][2], piece[i][3], 0, 1, 2, 3, 4, 5, 6, 7);
        }
    };

    Frags f0, f1;
    fetch(0, f0);
    // Steps 2p and 2p + 1.
    for (int p = 0; p < np; ++p) {
        const int s = 2 * p;
        fence();
        if constexpr (kDeep)
            wait_vmcnt<kXIssue + kWIssue>();
        else
            wait_vmcnt<0>();
        fence();
        even_step(s, f0, f1, staged(p + 1));
        __builtin_amdgcn_sched_barrier(0);  // the step's MFMAs stay ahead of the barrier
        fence();
        if constexpr (kDeep) wait_vmcnt<kWIssue>();
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();
        fence();
        if constexpr (kDeep) {
            issue_x(p + 2);
            order();
            load(p + 3);
            order();
        } else if (p + 2 < np) {
            load(p + 2);
        }
        fetch(s + 2, f0);  // past the last step: unused registers
        mfmas(f1);
        schedule();
        __builtin_amdgcn_sched_barrier(0);
    }

    // Epilogue. Block (i, j): lane holds out[m][n] for m = j-block row l%32 and, per register
    // r, n = i-block column 8·(r/4) + 4·(l/32) + r%4.
    fence();
    wait_vmcnt<0>();
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    fence();
    const float gxw = kMode == kW4A4 ? __fmul_rn(gx[0], gw[0]) : gw[0];
    const int nl = wn * kHalfN + 4 * fq;  // the lane's first column within the tile
#pragma unroll
    for (int i = 0; i < kNI; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int c = nl + i * 32 + 8 * g;
            float4 f = make_float4(gxw, gxw, gxw, gxw);
            if (kMode == kW4A4 && cs != nullptr) {
                const float4 cv = *reinterpret_cast<const float4*>(lds + kWsOff + 4 * c);
                f = make_float4(__fmul_rn(gxw, cv.x), __fmul_rn(gxw, cv.y), __fmul_rn(gxw, cv.z), __fmul_rn(gxw, cv.w));
            }
            const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[i][j][4 * g + r] = __fmul_rn(acc[i][j][4 * g + r], fv[r]);
        }

    // kW4A4: the low-rank term into the same accumulators: A = up rows (the tile's columns), B =
    // la rows, 16 ranks a call.
    if constexpr (kMode == kW4A4) {
        const auto upr = rows_view(up + static_cast<int64_t>(n0) * R, N - n0, 2 * R);
        const auto lar = rows_view(la + static_cast<int64_t>(m0) * R, padded_rows(M) - m0, 2 * R);
        for (int kk = 0; kk < R; kk += 16) {
            bf16x8 ua[4], lb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t ou = static_cast<uint32_t>(2 * ((wn * kHalfN + min(i, kNI - 1) * 32 + fr) * R + kk + 8 * fq));
                const uint32_t ol = static_cast<uint32_t>(2 * ((wm * 128 + i * 32 + fr) * R + kk + 8 * fq));
                if (i < kNI) ua[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(upr, ou, 0, 0));
                lb[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(lar, ol, 0, 0));
            }
#pragma unroll
            for (int i = 0; i < kNI; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ua[i], lb[j], acc[i][j], 0, 0, 0);
        }
    }

    uint2 bv[kNI][4];
    const bool has_bias = bias != nullptr;
#pragma unroll
    for (int i = 0; i < kNI; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            bv[i][g] = has_bias ? *reinterpret_cast<const uint2*>(lds + kBiasOff + 2 * (nl + i * 32 + 8 * g))
                                : make_uint2(0, 0);
    // Block row j at a time: computed and staged, then stored as whole rows (kHalfN = 96: 12 of
    // each row's 16 lanes).
    uint8_t* stage = lds + wave * kStageBytes;
    const int cl = (lane & 15) * 8;  // first of the lane's 8 columns in a stored row
    const int n = n0 + wn * kHalfN + cl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ml = j * 32 + fr;
#pragma unroll
        for (int i = 0; i < kNI; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = acc[i][j][4 * g + r];
                if (has_bias) {
                    v[0] = __fadd_rn(v[0], low_of<kOutHalf>(bv[i][g].x));
                    v[1] = __fadd_rn(v[1], high_of<kOutHalf>(bv[i][g].x));
                    v[2] = __fadd_rn(v[2], low_of<kOutHalf>(bv[i][g].y));
                    v[3] = __fadd_rn(v[3], high_of<kOutHalf>(bv[i][g].y));
                }
                const int col = i * 32 + 8 * g + 4 * fq;
                *reinterpret_cast<uint2*>(stage + ml * kStageRow + 2 * col) =
                    make_uint2(round2<kOutHalf>(v[0], v[1]), round2<kOutHalf>(v[2], v[3]));
            }
        wait_lgkmcnt0();  // a wave reads back only its own rows
#pragma unroll
        for (int r0 = 0; r0 < 32; r0 += 4) {
            const int rl = j * 32 + r0 + (lane >> 4);
            const int m = m0 + wm * 128 + rl;
            const uint4 v = *reinterpret_cast<const uint4*>(stage + rl * kStageRow + 2 * cl);
            if (m < M && n < N && cl < kHalfN) *reinterpret_cast<uint4*>(out + static_cast<int64_t>(m) * N + n) = v;
        }
    }
}

// Test entry: the quantizer's code conversion of values taken as quotients (scale·g = 1), two
// codes a byte (the first in the low nibble).
__global__ void e2m1_probe_kernel(const float* in, uint8_t* out, int64_t pairs) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= pairs) return;
    out[i] = static_cast<uint8_t>(
        put_e2m1_pair<0>(0u, e2m1_quotient(in[2 * i], 1.0f, 1.0f), e2m1_quotient(in[2 * i + 1], 1.0f, 1.0f)));
}

}  // namespace

int svdq_nvfp4_padded_rows(int M) { return padded_rows(M); }

hipError_t e2m1_probe(const float* in, uint8_t* out, int64_t n, hipStream_t s) {
    const int64_t pairs = n / 2;
    if (pairs == 0) return hipSuccess;
    e2m1_probe_kernel<<<static_cast<unsigned>((pairs + 255) / 256), 256, 0, s>>>(in, out, pairs);
    return hipGetLastError();
}

hipError_t svdq_nvfp4_input_scale(const void* x, bool x_half, const float* p, int M, int K,
                                  float* g, hipStream_t s) {
    uint32_t* word = reinterpret_cast<uint32_t*>(g);
    input_scale_init<<<1, 1, 0, s>>>(word);
    if (M == 0) return hipGetLastError();
    // ~256 workgroups (one a CU): the column chunks' workgroups times enough row slots.
    const int gx = (K / 8 + kScaleThreads - 1) / kScaleThreads;
    const int runs = (M + kScaleGroups * kScaleRows - 1) / (kScaleGroups * kScaleRows);
    const dim3 grid(gx, min(runs, max(1, 256 / gx)));
    constexpr int threads = kScaleThreads * kScaleGroups;
    if (x_half)
        input_scale_kernel<true><<<grid, threads, 0, s>>>(static_cast<const uint16_t*>(x), p, M, K, word);
    else
        input_scale_kernel<false><<<grid, threads, 0, s>>>(static_cast<const uint16_t*>(x), p, M, K, word);
    return hipGetLastError();
}

hipError_t svdq_nvfp4_quantize(const void* x, bool x_half, const float* p, const float* g,
                               const void* down, uint8_t* act, uint8_t* ascales, void* la, int M,
                               int K, int R, hipStream_t s) {
    if (M == 0) return hipSuccess;
#define COZYQ_RANK(RR)                                                                          \
    if (R == RR)                                                                                \
        return x_half ? launch_quantize<true, RR>(x, p, g, down, act, ascales, la, M, K, s)     \
                      : launch_quantize<false, RR>(x, p, g, down, act, ascales, la, M, K, s);
    COZYQ_RANK(32)
    COZYQ_RANK(64)
    COZYQ_RANK(128)
#undef COZYQ_RANK
    return hipErrorInvalidValue;
}

hipError_t svdq_nvfp4_gemm(const uint8_t* act, const uint8_t* ascales, const uint8_t* w,
                           const uint8_t* wscales, const float* gx, const float* gw,
                           const float* c, const void* la, const void* up, const void* bias,
                           void* out, bool out_half, int M, int N, int K, int R, hipStream_t s) {
    const bool wide = wide_tile(M, N);  // 256x192 tiles where they fill the CUs in fewer rounds
    const int tiles_m = (M + kTile - 1) / kTile, tiles_n = wide ? (N + 191) / 192 : (N + kTile - 1) / kTile;
    auto go = [&](auto kernel) {
        kernel<<<tiles_m * tiles_n, kThreads, 0, s>>>(
            act, ascales, w, wscales, gx, gw, c, static_cast<const uint16_t*>(la),
            static_cast<const uint16_t*>(up), static_cast<const uint16_t*>(bias),
            static_cast<uint16_t*>(out), M, N, K, R, tiles_m, tiles_n);
        return hipGetLastError();
    };
    if (wide)
        return out_half ? go(nvfp4_gemm_kernel<kW4A4, true, true, 192>) : go(nvfp4_gemm_kernel<kW4A4, true, false, 192>);
    return out_half ? go(nvfp4_gemm_kernel<kW4A4, true, true>) : go(nvfp4_gemm_kernel<kW4A4, true, false>);
}

hipError_t nvfp4_gemm(const void* x, bool x_half, const uint8_t* w, const uint8_t* scale,
                      const float* scale_2, const void* bias, void* out, bool out_half, int M, int N,
                      int K, hipStream_t s) {
    const int tiles_m = (M + kTile - 1) / kTile, tiles_n = (N + kTile - 1) / kTile;
    auto go = [&](auto kernel) {
        kernel<<<tiles_m * tiles_n, kThreads, 0, s>>>(
            static_cast<const uint8_t*>(x), nullptr, w, scale, nullptr, scale_2, nullptr, nullptr,
            nullptr, static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), M, N, K, 0,
            tiles_m, tiles_n);
        return hipGetLastError();
    };
    if (x_half)
        return out_half ? go(nvfp4_gemm_kernel<kW4A16, true, true>) : go(nvfp4_gemm_kernel<kW4A16, true, false>);
    return out_half ? go(nvfp4_gemm_kernel<kW4A16, false, true>) : go(nvfp4_gemm_kernel<kW4A16, false, false>);
}

}  // namespace cozyq
