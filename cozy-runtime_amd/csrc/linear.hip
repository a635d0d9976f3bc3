// The fused int8 linear: block-Hadamard rotation, per-token int8 quantization and the W8A8 GEMM
// with its dequantizing epilogue, in one persistent launch.
//
// The reference runs the producer and the GEMM as two launches chained by programmatic
// dependent launch (kernels/csrc/gemm/rotate.cu:284-295, gemm_tma.cuh:166-173). Here both are
// jobs of one kernel. Per-token scaling needs a whole row's maximum before any of the row's
// codes exist, so the rows are quantized once into `q` / `qs` (which the caller may keep as the
// shared operand) and every output tile of an M-tile waits for that M-tile's rows. The wait is on
// a counter the quantize jobs raise.
//
// Work is split into `queues` job queues (one per XCD when workgroup b runs on XCD b mod 8, the
// dispatch order on MI355X). Queue x owns M-tiles m with m mod queues == x:
// - first the quantize jobs of all of them: 16 rows each, two a wave (rows.h);
// - then their output tiles, pair of M-tiles by pair, N fastest with the two M-tiles
//   alternating, so an XCD's concurrent tiles share two X panels and their W panels in its L2.
// A workgroup claims the next job of its queue with an atomic counter. Before its first tile it
// waits for its queue's quantize jobs, all claimed before any tile by running workgroups that
// never wait themselves, so every wait ends. A spin limit guards the wait anyway: past it the
// workgroup records the fault and writes NaN into every output tile it claims instead of
// computing it from codes that may not exist yet, so no tile is ever silently wrong.
//
// The workspace (kernels.h `linear_workspace_ints`) holds the queue heads, an exit count, the
// fault flag, a status word and one done-counter per M-tile. It must be zero before the first
// launch. The last workgroup to leave moves the fault flag into the status word and sets every
// counter back to zero, so the next launch on the stream starts clean; the status word stays set
// until the host reads it (linear_status). Launches that overlap on one workspace race.
#include "gemm_tile.h"
#include "rows.h"

namespace cozyq {
namespace {

constexpr int kQRows = 16;          // rows a quantize job takes: 2 a wave
constexpr int kMaxQueues = 8;       // XCDs on MI355X
constexpr int kSpinLimit = 1 << 24;  // s_sleep(2) rounds a tile waits at most (~1 s)
constexpr int kJobSlot = kLdsBytes8;  // LDS word that broadcasts a claimed job
constexpr int kFusedLds = kLdsBytes8 + 16;
constexpr int kQWaveRows = kQRows / (kThreads8 / 64);  // a wave's rows of a quantize job
static_assert(kThreads8 / 64 * kRowLdsFloats<128> * 4 <= kLdsBytes8 &&
                  kThreads8 / 64 * kRowLdsFloats<256> * 4 <= kLdsBytes8,
              "every wave's rotation slice fits the tile's LDS");

// Workspace layout (int32): [0, 8) queue heads, [8] exit count, [9] fault flag (this launch),
// [10] status (a launch since the last read gave up a wait), [16, 16 + tiles_m) quantize jobs
// finished per M-tile.
constexpr int kExit = 8, kFault = 9, kStatus = 10, kDone = 16;

// The spin limit launches use: kSpinLimit, or what the test hook set (a negative value makes
// every wait give up at once, which exercises the fault path without any wave waiting).
int spin_limit_setting = kSpinLimit;

__device__ __forceinline__ int qjobs(int m, int M) {
    const int rows = min(kTile, M - m * kTile);
    return (rows + kQRows - 1) / kQRows;
}

// Job `j` of queue `x`: kind (0 quantize, 1 tile), M-tile and the index within the kind.
struct Job {
    int kind, m, index, n;
};

__device__ __forceinline__ int queue_jobs(int x, int queues, int tiles_m, int tiles_n, int M) {
    int total = 0;
    for (int m = x; m < tiles_m; m += queues) total += qjobs(m, M) + tiles_n;
    return total;
}

__device__ __forceinline__ Job decode(int j, int x, int queues, int tiles_m, int tiles_n, int M) {
    // The queue's quantize jobs first, M-tile by M-tile; then its tiles, pair of M-tiles by pair,
    // N fastest with the two M-tiles alternating.
    for (int m = x; m < tiles_m; m += queues) {
        const int n = qjobs(m, M);
        if (j < n) return {0, m, j, 0};
        j -= n;
    }
    for (int m = x; m < tiles_m; m += 2 * queues) {
        const int m2 = m + queues;
        const bool pair = m2 < tiles_m;
        const int tiles = (pair ? 2 : 1) * tiles_n;
        if (j < tiles) return {1, pair && (j & 1) ? m2 : m, 0, pair ? j >> 1 : j};
        j -= tiles;
    }
    return {-1, 0, 0, 0};
}

// A wave's rows r0 .. r0 + kQWaveRows - 1 of a quantize job (rows past M skipped), their loads
// issued up front: one load latency for the job instead of one a row.
template <bool kHalf, int kRot>
__device__ __forceinline__ void quantize_job(const uint16_t* __restrict__ x, int8_t* __restrict__ q,
                                                       float* __restrict__ qs, int M, int K, int r0, int lane,
                                                       float* slice) {
    constexpr int kWaveRows = kQWaveRows;
    const int rows = min(kWaveRows, M - r0);
    uint4 raw[kWaveRows][kRowLoads];
#pragma unroll
    for (int i = 0; i < kWaveRows; ++i)
        row_loads(row_view(x + static_cast<int64_t>(min(r0 + i, M - 1)) * K, K), lane, raw[i]);
#pragma unroll
    for (int i = 0; i < kWaveRows; ++i)
        if (i < rows)
            quantize_row_wave<kHalf, kRot>(raw[i], K, lane, slice, q + static_cast<int64_t>(r0 + i) * K, qs + r0 + i);
}

// Output tile (tm, tn) filled with the output dtype's NaN: what a workgroup whose wait gave up
// writes in place of the tile.
template <bool kOutHalf>
__device__ __forceinline__ void nan_tile(uint16_t* __restrict__ out, int64_t ldo, int M, int N, int tm, int tn) {
    const uint16_t nan = kOutHalf ? 0x7e00 : 0x7fc0;
    const int m0 = tm * kTile, n0 = tn * kTile;
    const int rows = min(kTile, M - m0), cols = min(kTile, N - n0);
    for (int i = threadIdx.x; i < rows * cols; i += blockDim.x)
        out[static_cast<int64_t>(m0 + i / cols) * ldo + n0 + i % cols] = nan;
}

template <bool kHalf, int kRot, bool kOutHalf, bool kBias, int kEpi>
__global__ __launch_bounds__(kThreads8, 1) void linear_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ qs,
    const int8_t* __restrict__ W, const float* __restrict__ ws, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ out, int64_t ldo, int M, int N, int K, int tiles_m, int tiles_n,
    int queues, int* __restrict__ work, int spin_limit) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kFusedLds];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qx = blockIdx.x % queues;
    const int total = queue_jobs(qx, queues, tiles_m, tiles_n, M);
    int* done = work + kDone;
    bool acquired = false;  // the queue's rows, once all are quantized
    bool faulted = false;   // the wait for them gave up: tiles are written as NaN
    for (;;) {
        if (tid == 0)
            *reinterpret_cast<int*>(lds + kJobSlot) =
                __hip_atomic_fetch_add(work + qx, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();  // also: every wave is done with the LDS of the job before
        const int j = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const int*>(lds + kJobSlot));
        if (j >= total) break;
        const Job job = decode(j, qx, queues, tiles_m, tiles_n, M);
        if (job.kind == 0) {
            quantize_job<kHalf, kRot>(x, q, qs, M, K, job.m * kTile + job.index * kQRows + wave * kQWaveRows,
                                      lane, reinterpret_cast<float*>(lds) + wave * kRowLdsFloats<kRot>);
            // Every wave's codes and scales have reached L2 before the barrier; then one
            // agent-scope release (a write-back of the XCD's L2) publishes the job.
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            __syncthreads();
            if (tid == 0) __hip_atomic_fetch_add(done + job.m, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            continue;
        }
        // Before its first tile a workgroup waits for every quantize job of its queue (all
        // claimed before any tile, by running workgroups that never wait) and acquires their
        // rows once: an agent-scope acquire invalidates the XCD's L2, so it is taken before the
        // tiles start filling it, not per tile.
        if (!acquired) {
            if (tid == 0) {
                int spins = 0;
                bool gave_up = spin_limit < 0;
                for (int m = qx; m < tiles_m && !gave_up; m += queues) {
                    const int need = qjobs(m, M);
                    while (__hip_atomic_load(done + m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < need) {
                        __builtin_amdgcn_s_sleep(2);
                        if (++spins >= spin_limit) {
                            gave_up = true;
                            break;
                        }
                    }
                }
                if (gave_up) __hip_atomic_store(work + kFault, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                *reinterpret_cast<int*>(lds + kJobSlot + 4) = gave_up;
            }
            __syncthreads();
            faulted = *reinterpret_cast<const int*>(lds + kJobSlot + 4) != 0;
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            acquired = true;
        }
        if (faulted) {
            nan_tile<kOutHalf>(out, ldo, M, N, job.m, job.n);
            continue;
        }
        gemm_tile8<kInt8, kOutHalf, kBias, kEpi>(
            lds, reinterpret_cast<const uint8_t*>(q), reinterpret_cast<const uint8_t*>(W), qs, ws,
            bias, out, ldo, M, N, K, job.m, job.n);
    }
    // The last workgroup out moves the fault flag into the status word and resets the counters
    // for the next launch. Every workgroup's fault store precedes its exit increment, which the
    // last one's acquire sees.
    if (tid == 0) {
        const int before = __hip_atomic_fetch_add(work + kExit, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (before == static_cast<int>(gridDim.x) - 1) {
            if (__hip_atomic_load(work + kFault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                __hip_atomic_store(work + kStatus, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(work + kFault, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            for (int i = 0; i < kMaxQueues; ++i) __hip_atomic_store(work + i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int m = 0; m < tiles_m; ++m) __hip_atomic_store(done + m, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(work + kExit, 0, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <bool kHalf, int kRot, bool kOutHalf, bool kBias, int kEpi>
hipError_t launch_linear(const void* x, int8_t* q, float* qs, const int8_t* w, const float* ws,
                         const void* bias, void* out, int64_t ldo, int M, int N, int K, int* work,
                         int device, hipStream_t s) {
    const int tiles_m = (M + kTile - 1) / kTile, tiles_n = (N + kTile - 1) / kTile;
    const int queues = min(kMaxQueues, tiles_m);
    int jobs = 0;
    for (int m = 0; m < tiles_m; ++m) jobs += (min(kTile, M - m * kTile) + kQRows - 1) / kQRows + tiles_n;
    const int grid = max(queues, min(cu_count(device), jobs));
    linear_kernel<kHalf, kRot, kOutHalf, kBias, kEpi><<<grid, kThreads8, 0, s>>>(
        static_cast<const uint16_t*>(x), q, qs, w, ws, static_cast<const uint16_t*>(bias),
        static_cast<uint16_t*>(out), ldo, M, N, K, tiles_m, tiles_n, queues, work, spin_limit_setting);
    return hipGetLastError();
}

// The allocation-free variant's counters: a file-scope device array, one per GPU the library
// runs on, held until the process ends. Host code never passes the array's name to a kernel (it
// is a host-side stand-in there); it passes the device address hipGetSymbolAddress gives, taken
// once per device with that device current.
constexpr int kScratchInts = kDone + 1024;  // up to 1024 M-tiles: M <= 262144
__device__ __align__(256) int scratch[kScratchInts];

int* scratch_address[64] = {nullptr};

hipError_t scratch_of(int device, int** out) {
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    if (scratch_address[device] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        scratch_address[device] = static_cast<int*>(p);
    }
    *out = scratch_address[device];
    return hipSuccess;
}

// The counters a launch uses, set to zero on the launch's stream ahead of it (a kernel, not a
// memset node, so a captured graph replays it correctly). The status word is cleared with them:
// the allocation-free entry point's status describes its last call.
__global__ __launch_bounds__(256) void clear_ints(int* __restrict__ p, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

}  // namespace

int cu_count(int device) {
    static int counts[64] = {0};
    if (device < 0 || device >= 64) return 256;
    if (counts[device] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n <= 0) n = 256;
        counts[device] = n;
    }
    return counts[device];
}

int linear_workspace_ints(int M) { return kDone + (M + kTile - 1) / kTile; }

hipError_t linear_int8(const void* x, bool half, int rotation, int8_t* q, float* qs, const int8_t* w,
                       const float* ws, const void* bias, void* out, int64_t ldo, int M, int N, int K,
                       int epilogue, int* work, int device, hipStream_t s) {
    if (M == 0 || N == 0) return hipSuccess;
    const bool b = bias != nullptr;
#define COZYQ_LIN(H, R, B, E)                                                                     \
    if (half == H && rotation == R && b == B && epilogue == E)                                     \
        return launch_linear<H, R, H, B, E>(x, q, qs, w, ws, bias, out, ldo, M, N, K, work, device, s);
#define COZYQ_LIN_R(H, B, E) COZYQ_LIN(H, 256, B, E) COZYQ_LIN(H, 128, B, E) COZYQ_LIN(H, 0, B, E)
    COZYQ_LIN_R(false, false, 0)
    COZYQ_LIN_R(false, true, 0)
    COZYQ_LIN_R(false, false, 1)
    COZYQ_LIN_R(false, true, 1)
    COZYQ_LIN_R(true, false, 0)
    COZYQ_LIN_R(true, true, 0)
    COZYQ_LIN_R(true, false, 1)
    COZYQ_LIN_R(true, true, 1)
#undef COZYQ_LIN_R
#undef COZYQ_LIN
    return hipErrorInvalidValue;
}

int linear_noalloc_max_rows() { return (kScratchInts - kDone) * kTile; }

hipError_t linear_status(int* work, int device, hipStream_t s, int* status) {
    if (work == nullptr) {
        const hipError_t e = scratch_of(device, &work);
        if (e != hipSuccess) return e;
    }
    int word = 0;
    hipError_t e = hipMemcpyAsync(&word, work + kStatus, sizeof(int), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return e;
    if (word != 0) {
        clear_ints<<<1, 64, 0, s>>>(work + kStatus, 1);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) return e;
    }
    *status = word;
    return hipSuccess;
}

void linear_set_spin_limit(int limit) { spin_limit_setting = limit == 0 ? kSpinLimit : limit; }

hipError_t linear_int8_noalloc(const void* x, bool half, int rotation, int8_t* q, float* qs,
                               const int8_t* w, const float* ws, const void* bias, void* out,
                               int64_t ldo, int M, int N, int K, int epilogue, int device,
                               hipStream_t s) {
    if (M > linear_noalloc_max_rows()) return hipErrorInvalidValue;
    if (M == 0 || N == 0) return hipSuccess;
    int* counters = nullptr;
    const hipError_t e = scratch_of(device, &counters);
    if (e != hipSuccess) return e;
    clear_ints<<<1, 256, 0, s>>>(counters, linear_workspace_ints(M));
    const hipError_t launched = hipGetLastError();
    if (launched != hipSuccess) return launched;
    return linear_int8(x, half, rotation, q, qs, w, ws, bias, out, ldo, M, N, K, epilogue, counters, device, s);
}

}  // namespace cozyq
