// The W8A8 int8 GEMM on gfx950: out = epilogue(q · wᵀ), q [M, K] and w [N, K] int8, exact int32
// accumulation on v_mfma_i32_32x32x32_i8 (from one wave per SIMD it sustains 82% of the int8
// peak where the 16x16x64 form sustains 53%, measured on MI355X).
//
// A workgroup of 4 waves owns a 256x256 output tile; each wave a 128x128 quadrant as 4x4 MFMA
// blocks of 32x32 (256 accumulator registers a lane, held in AGPRs). K advances 64 bytes a step through a
// ring of 4 LDS slots (32 KB each: the X and W tiles' 256 rows x 64 bytes), filled by
// buffer_load_dwordx4 ... lds straight from HBM/L2 — no staging registers, and rows past M or N
// and columns past K read as zeros through the buffer's bounds. A slot is refilled three steps
// before it is read, one barrier a step; each step's MFMAs run on fragments read from LDS during
// the previous step. Tiles are ordered so that each XCD (workgroups b ≡ x mod 8) works through a
// contiguous run of tiles, 4 M-tiles by 8 N-tiles at a time, which share their X and W K-slices
// in that XCD's L2.
#include "common.h"
#include "kernels.h"

namespace cozyq {
namespace {

constexpr int kTile = 256;
constexpr int kSlotK = 64;                     // K bytes per slot
constexpr int kSlots = 4;
constexpr int kThreads = 256;
constexpr int kOpBytes = kTile * kSlotK;       // one operand's slot: 16 KB
constexpr int kSlotBytes = 2 * kOpBytes;       // X then W
constexpr int kLoadsPerSlot = 8;               // buffer loads a lane issues per slot
constexpr uint32_t kOutOfRange = 0x80000000u;  // a buffer offset past num_records reads zeros
constexpr int kGroupM = 4;                     // M-tiles a tile group spans

constexpr int kStageRow = 128 * 2 + 16;         // one staged output row: 128 bf16 + pad
constexpr int kStageBytes = 128 * kStageRow;    // one wave's staged quadrant
constexpr int kLdsBytes = 4 * kStageBytes > kSlots * kSlotBytes ? 4 * kStageBytes : kSlots * kSlotBytes;

typedef __attribute__((address_space(3))) void LdsPtr;
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

// s_waitcnt with only vmcnt <= N (expcnt and lgkmcnt left unconstrained): gfx9 encoding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Keeps the compiler from moving memory operations across the waits and barriers below.
__device__ __forceinline__ void fence() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ void wait_lgkmcnt0() {
    __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));
}

// 16-byte chunk `c` (0..3) of LDS row `r` sits at chunk c ^ ((r/2) % 4): any 8 consecutive rows
// read at one chunk land on 8 distinct 16-byte bank groups of a 128-byte LDS cycle (measured
// conflict-free on gfx950 with SQ_LDS_BANK_CONFLICT).
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 3); }

__device__ __forceinline__ float gelu_tanh(float y) {
    // 0.5·y·(1 + tanh(u)) = y / (1 + e^(-2u)), u = 0.79788456·(y + 0.044715·y³); e^t as 2^(t·log2 e)
    const float u = 0.79788456f * (y + 0.044715f * y * y * y);
    return y * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-2.8853900817779268f * u));
}

template <bool kOutHalf>
__device__ __forceinline__ uint16_t round_out(float v) {
    if constexpr (kOutHalf) {
        return narrow<true>(v);
    } else {
        return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));  // v_cvt_pk_bf16_f32: RNE
    }
}

// kEpi: 0 the CPU law's dequantization (+ bias in the output dtype), 1 that then tanh-GELU,
// 2 the raw int32 accumulators (test entry).
template <bool kOutHalf, bool kBias, int kEpi>
__global__ __launch_bounds__(kThreads, 1) void gemm_i8_kernel(
    const int8_t* __restrict__ X, const int8_t* __restrict__ W, const float* __restrict__ xs,
    const float* __restrict__ ws, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out,
    int32_t* __restrict__ acc_out, int64_t ldo, int M, int N, int K, int tiles_m, int tiles_n) {
    // The ring during the K loop; afterwards each wave's 128x128 output quadrant, staged for
    // whole-row stores (rows padded to kStageRow bytes).
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kLdsBytes];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS-DMA bases go in M0
    const int wm = wave >> 1, wn = wave & 1;

    // Tile order: XCD-contiguous runs, then groups of kGroupM M-tiles with N fastest inside.
    const int tiles = tiles_m * tiles_n;
    int t = blockIdx.x;
    if ((tiles & 7) == 0) t = (t & 7) * (tiles >> 3) + (t >> 3);
    const int group = t / (kGroupM * tiles_n);
    const int gm = min(kGroupM, tiles_m - group * kGroupM);
    const int within = t - group * kGroupM * tiles_n;
    const int tm = group * kGroupM + within % gm, tn = within / gm;
    // The tile arithmetic divides on the vector unit; the origin is uniform, and buffer
    // descriptors must sit in scalar registers.
    const int m0 = __builtin_amdgcn_readfirstlane(tm * kTile);
    const int n0 = __builtin_amdgcn_readfirstlane(tn * kTile);

    // Buffer views of this tile's rows: reads past the last row return zeros.
    const int64_t xspan = static_cast<int64_t>(M - m0) * K, wspan = static_cast<int64_t>(N - n0) * K;
    const uint32_t xbytes = xspan > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(xspan);
    const uint32_t wbytes = wspan > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(wspan);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(X + static_cast<int64_t>(m0) * K), 0, xbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(W + static_cast<int64_t>(n0) * K), 0, wbytes, 0x00020000);

    // Load j (0..3) of a wave fills LDS rows [(4j + wave)·16, +16) of an operand's slot: lane l
    // writes row +l/4, physical chunk l%4, so it reads that row's logical chunk (l%4) ^ swz.
    int rowoff[4], chunk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = (4 * j + wave) * 16 + (lane >> 2);
        chunk[j] = 16 * swz(r, lane & 3);
        rowoff[j] = r * K + chunk[j];
    }
#define COZYQ_ISSUE(step)                                                                            \
    do {                                                                                             \
        uint8_t* slot_ = lds + ((step) & (kSlots - 1)) * kSlotBytes;                                                \
        const int k0_ = (step) * kSlotK;                                                             \
        _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                              \
            const uint32_t off_ = (k0_ + chunk[j] < K) ? static_cast<uint32_t>(rowoff[j] + k0_) : kOutOfRange; \
            const int base_ = (4 * j + wave) * 1024;                                                 \
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (LdsPtr*)(slot_ + base_), 16, off_, 0, 0, 0); \
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (LdsPtr*)(slot_ + kOpBytes + base_), 16, off_, 0, 0, 0); \
        }                                                                                            \
    } while (0)

    // Fragment reads (32x32x32: lane l supplies row l%32, 16-byte chunk l/32 of a 32-byte K
    // half): A = W rows (wn half), B = X rows (wm half); two K halves a slot.
    const int fr = lane & 31, fq = lane >> 5;
    int aoff[2][4], boff[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rw = wn * 128 + i * 32 + fr, rx = wm * 128 + i * 32 + fr;
            aoff[h][i] = kOpBytes + rw * kSlotK + 16 * swz(rw, 2 * h + fq);
            boff[h][i] = rx * kSlotK + 16 * swz(rx, 2 * h + fq);
        }
    auto fetch = [&](int step, i32x4 (*a)[4], i32x4 (*b)[4]) {
        const uint8_t* slot = lds + (step & (kSlots - 1)) * kSlotBytes;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a[h][i] = *reinterpret_cast<const i32x4*>(slot + aoff[h][i]);
                b[h][i] = *reinterpret_cast<const i32x4*>(slot + boff[h][i]);
            }
    };

    i32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    const int nk = (K + kSlotK - 1) / kSlotK;
    // Every step issues one slot's loads, also past the last step (their offsets fall outside
    // the buffer: no traffic, zeros into a slot nothing reads), so each step is one block the
    // scheduler can interleave and the pending-load count at a step's top is always two slots.
#pragma unroll
    for (int s = 0; s < kSlots; ++s) COZYQ_ISSUE(s);
    fence();
    wait_vmcnt<3 * kLoadsPerSlot>();  // slot 0 complete
    __builtin_amdgcn_s_barrier();
    fence();

    i32x4 fa[2][2][4], fb[2][2][4];
    fetch(0, fa[0], fb[0]);

    auto step_body = [&](int s, i32x4 (*ca)[4], i32x4 (*cb)[4], i32x4 (*na)[4], i32x4 (*nb)[4]) {
        fence();
        wait_vmcnt<2 * kLoadsPerSlot>();  // slot s+1 complete (s+2 and s+3 may be in flight)
        wait_lgkmcnt0();                  // this wave's reads of slot s are in registers
        __builtin_amdgcn_s_barrier();     // every wave's are: slot s may be refilled
        fence();
        COZYQ_ISSUE(s + kSlots);
        fetch(s + 1, na, nb);  // past the last step: unused registers
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ca[h][i], cb[h][j], acc[i][j], 0, 0, 0);
        // Issue order: the step's 8 slot loads first, then one fragment read per two MFMAs.
        // Loads spread between the MFMAs stall the wave (and its matrix core) whenever the
        // memory queue is full; issued up front they queue while the MFMAs run (measured on
        // MI355X: 218 -> 187 us at config 2 against the spread order).
        __builtin_amdgcn_sched_group_barrier(0x020, 8, 0);      // 8 buffer loads (to LDS)
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // 2 MFMA
        }
    };
    int s = 0;
    for (; s + 1 < nk; s += 2) {
        step_body(s, fa[0], fb[0], fa[1], fb[1]);
        step_body(s + 1, fa[1], fb[1], fa[0], fb[0]);
    }
    if (s < nk) step_body(s, fa[0], fb[0], fa[1], fb[1]);

    // Epilogue. Block (i, j): lane holds out[m][n] for m = j-block row l%32 and, per register
    // r, n = i-block column 8·(r/4) + 4·(l/32) + r%4 (MFMA rows are W rows): four runs of four
    // consecutive columns, each an 8-byte store. The lane's 64 weight scales and biases are
    // loaded once, ahead of the arithmetic.
    const int nl = n0 + wn * 128 + 4 * fq;  // the lane's first column
    if constexpr (kEpi == 2) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = m0 + wm * 128 + j * 32 + fr;
            if (m >= M) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i)
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
    float4 wsv[4][4];
    uint2 bv[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = min(nl + i * 32 + 8 * g, N - 4);  // N % 8 == 0: a clamped run stays in bounds
            wsv[i][g] = *reinterpret_cast<const float4*>(ws + n);
            if constexpr (kBias) bv[i][g] = *reinterpret_cast<const uint2*>(bias + n);
        }
    // All loads have landed and all waves are done with the ring before it becomes the staging
    // area.
    fence();
    wait_vmcnt<0>();
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    fence();
    uint8_t* stage = lds + wave * kStageBytes;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ml = j * 32 + fr;  // row within the quadrant
        const int m = m0 + wm * 128 + ml;
        const float xsm = xs[min(m, M - 1)];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float w4[4] = {wsv[i][g].x, wsv[i][g].y, wsv[i][g].z, wsv[i][g].w};
                uint16_t b4[4] = {0, 0, 0, 0};
                if constexpr (kBias) {
                    b4[0] = bv[i][g].x & 0xffff; b4[1] = bv[i][g].x >> 16;
                    b4[2] = bv[i][g].y & 0xffff; b4[3] = bv[i][g].y >> 16;
                }
                uint16_t o[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    // internal/int8_linear.py:445-448 then :276: (acc·xs)·ws rounded to float32
                    // at each product, one cast, then + bias in the output dtype.
                    const float v = __fmul_rn(__fmul_rn(static_cast<float>(acc[i][j][4 * g + r]), xsm), w4[r]);
                    o[r] = round_out<kOutHalf>(v);
                    if constexpr (kBias)
                        o[r] = round_out<kOutHalf>(__fadd_rn(widen<kOutHalf>(o[r]), widen<kOutHalf>(b4[r])));
                    if constexpr (kEpi == 1) o[r] = round_out<kOutHalf>(gelu_tanh(widen<kOutHalf>(o[r])));
                }
                const int col = i * 32 + 8 * g + 4 * fq;  // column within the quadrant
                *reinterpret_cast<uint2*>(stage + ml * kStageRow + 2 * col) =
                    make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16), o[2] | (static_cast<uint32_t>(o[3]) << 16));
            }
    }
    wait_lgkmcnt0();  // a wave reads back only its own quadrant
    // Whole rows: 16 lanes cover one quadrant row's 256 bytes; 4 rows an instruction.
    const int cl = (lane & 15) * 8;  // first of the lane's 8 columns
    const int n = n0 + wn * 128 + cl;
#pragma unroll 4
    for (int r0 = 0; r0 < 128; r0 += 4) {
        const int ml = r0 + (lane >> 4);
        const int m = m0 + wm * 128 + ml;
        const uint4 v = *reinterpret_cast<const uint4*>(stage + ml * kStageRow + 2 * cl);
        if (m < M && n < N) *reinterpret_cast<uint4*>(out + static_cast<int64_t>(m) * ldo + n) = v;
    }
}

#undef COZYQ_ISSUE

template <bool kOutHalf, bool kBias, int kEpi>
hipError_t launch(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                  const void* bias, void* out, int32_t* acc, int64_t ldo, int M, int N, int K,
                  hipStream_t s) {
    const int tiles_m = (M + kTile - 1) / kTile, tiles_n = (N + kTile - 1) / kTile;
    gemm_i8_kernel<kOutHalf, kBias, kEpi><<<tiles_m * tiles_n, kThreads, 0, s>>>(
        q, w, xs, ws, static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), acc, ldo,
        M, N, K, tiles_m, tiles_n);
    return hipGetLastError();
}

}  // namespace

hipError_t gemm_int8(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                     const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                     int epilogue, hipStream_t s) {
    if (M <= 256)  // few rows: narrow tiles keep ~224 workgroups on the weight stream
        return gemm_int8_narrow(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s);
    const bool b = bias != nullptr;
#define COZYQ_CASE(H, B, E) \
    if (out_half == H && b == B && epilogue == E) return launch<H, B, E>(q, xs, w, ws, bias, out, nullptr, ldo, M, N, K, s);
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

hipError_t gemm_int8_acc(const int8_t* q, const int8_t* w, int32_t* acc, int M, int N, int K,
                         hipStream_t s) {
    return launch<false, false, 2>(q, nullptr, w, nullptr, nullptr, nullptr, acc, N, M, N, K, s);
}

}  // namespace cozyq
