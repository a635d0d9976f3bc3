// The C ABI of include/cozyq.h: argument checks, the device guard and the kernel dispatch.
// Shapes and modes are checked here (hipErrorInvalidValue, as kernels/csrc/gemm.cpp:81-97,
// 130-133 does); dtypes, contiguity and alignment are the Python caller's, as in the reference.
#include <hip/hip_runtime.h>

#include "../../include/cozyq.h"
#include "common.h"
#include "kernels.h"

namespace {

// `device` current for one call and the caller's restored after (kernels/csrc/gemm.cpp:22-39).
class OnDevice {
  public:
    explicit OnDevice(int device) {
        error_ = hipGetDevice(&previous_);
        if (error_ == hipSuccess && previous_ != device) error_ = hipSetDevice(device);
    }
    ~OnDevice() {
        int now = -1;
        if (error_ == hipSuccess && hipGetDevice(&now) == hipSuccess && now != previous_)
            (void)hipSetDevice(previous_);
    }
    hipError_t error() const { return error_; }

  private:
    int previous_ = -1;
    hipError_t error_ = hipSuccess;
};

hipStream_t on(void* stream) { return static_cast<hipStream_t>(stream); }

bool fits(int K, int multiple) { return K > 0 && K <= cozyq::kMaxK && K % multiple == 0; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

extern "C" {

int cozyq_not_supported(void) { return hipErrorNotSupported; }
int cozyq_out_of_memory(void) { return hipErrorOutOfMemory; }
int cozyq_gemv_rows(void) { return 4; }
int cozyq_max_k(void) { return cozyq::kMaxK; }
const char* cozyq_arch(void) { return "gfx950"; }
const char* cozyq_error_name(int code) { return hipGetErrorName(static_cast<hipError_t>(code)); }

int cozyq_quantize(int device, int fp8, const void* x, int x_half, void* q, float* scales, int M,
                   int K, const void* scale, const void* shift, int64_t scale_stride,
                   int64_t shift_stride, int rows_per_entry, int norm, float eps, int activation,
                   const void* up, void* stream) {
    if (!fits(K, fp8 ? 16 : 256) || M < 0 || norm < 0 || norm > 2 || activation < 0 ||
        activation > 4 || rows_per_entry < 1)
        return hipErrorInvalidValue;
    const bool gated = activation == 3 || activation == 4;
    if (gated && (norm != 0 || scale || shift)) return hipErrorInvalidValue;
    if (up != nullptr && activation != 4) return hipErrorInvalidValue;
    // The tables and `up` are read 16 bytes at a time, as x is.
    if ((scale && (!aligned16(scale) || scale_stride < 0 || scale_stride % 8)) ||
        (shift && (!aligned16(shift) || shift_stride < 0 || shift_stride % 8)) ||
        (up && !aligned16(up)) || !aligned16(x))
        return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    const cozyq::Prologue pro{static_cast<const uint16_t*>(scale), static_cast<const uint16_t*>(shift),
                              scale_stride, shift_stride, rows_per_entry, norm, eps, activation,
                              static_cast<const uint16_t*>(up)};
    const bool any = scale || shift || norm || activation;
    if (fp8)
        return cozyq::fp8_quantize(x, x_half, static_cast<uint8_t*>(q), scales, M, K,
                                   any ? &pro : nullptr, on(stream));
    return cozyq::rotate_quantize(x, x_half, static_cast<int8_t*>(q), scales, M, K, 256,
                                  any ? &pro : nullptr, on(stream));
}

int cozyq_quantize_rot(int device, const void* x, int x_half, int8_t* q, float* scales, int M,
                       int K, int rotation, void* stream) {
    const int multiple = rotation == 0 ? 16 : rotation;
    if ((rotation != 0 && rotation != 128 && rotation != 256) || !fits(K, multiple) || M < 0)
        return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::rotate_quantize(x, x_half, q, scales, M, K, rotation, nullptr, on(stream));
}

int cozyq_gemv(int device, const void* x, int x_half, const int8_t* w, const float* w_scale,
               const void* bias, void* out, int out_half, int M, int N, int K, void* stream) {
    if (!fits(K, 256) || N < 1 || M < 0) return hipErrorInvalidValue;
    // The kernel writes four outputs (8 bytes) a wave and reads 16 bytes a lane.
    if (N % 8 || !aligned16(x) || !aligned16(w) || (reinterpret_cast<uintptr_t>(out) & 7))
        return hipErrorNotSupported;
    if (M == 0) return hipSuccess;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::int8_linear_small(x, x_half, w, w_scale, bias, out, out_half, M, N, K,
                                    on(stream));
}

static int gemm_checked(int device, int fp8, const void* q, const float* scales, const void* w,
                        const float* w_scale, const void* bias, void* out, int64_t ldo,
                        int out_half, int M, int N, int K, int epilogue, int multiple,
                        int config, void* stream) {
    if (M < 1 || N < 1 || N % 8 || !fits(K, multiple) || epilogue < 0 || epilogue > 1)
        return hipErrorInvalidValue;
    if (ldo < N || ldo % 8 || !aligned16(out)) return hipErrorInvalidValue;
    if (config >= cozyq::kGemmConfigs) return hipErrorNotSupported;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    if (config < 0) config = -1;
    if (fp8)
        return cozyq::gemm_fp8(static_cast<const uint8_t*>(q), scales,
                               static_cast<const uint8_t*>(w), w_scale, bias, out, ldo, out_half,
                               M, N, K, epilogue, config, on(stream));
    return cozyq::gemm_int8(static_cast<const int8_t*>(q), scales, static_cast<const int8_t*>(w),
                            w_scale, bias, out, ldo, out_half, M, N, K, epilogue, config, on(stream));
}

static int linear_checked(int device, const void* x, int x_half, int rotation, int8_t* q,
                          float* qs, const int8_t* w, const float* w_scale, const void* bias,
                          void* out, int64_t ldo, int out_half, int M, int N, int K, int epilogue,
                          int* workspace, bool own_scratch, void* stream) {
    if (M < 0 || N < 1 || N % 8 || epilogue < 0 || epilogue > 1) return hipErrorInvalidValue;
    if (rotation != 0 && rotation != 128 && rotation != 256) return hipErrorInvalidValue;
    if (!fits(K, rotation == 0 ? 16 : rotation)) return hipErrorInvalidValue;
    if (ldo < N || ldo % 8 || !aligned16(out) || !aligned16(x) || !aligned16(q) || !aligned16(w))
        return hipErrorInvalidValue;
    if (M > 0 && (!qs || !w_scale || (!own_scratch && !workspace))) return hipErrorInvalidValue;
    if (own_scratch && M > cozyq::linear_noalloc_max_rows()) return hipErrorInvalidValue;
    // One wave quantizes a row, so rows longer than 4096 take the two-launch path; the output
    // is in x's dtype.
    if (K > 4096 || out_half != x_half) return hipErrorNotSupported;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    if (own_scratch)
        return cozyq::linear_int8_noalloc(x, x_half != 0, rotation, q, qs, w, w_scale, bias, out, ldo,
                                          M, N, K, epilogue, device, on(stream));
    return cozyq::linear_int8(x, x_half != 0, rotation, q, qs, w, w_scale, bias, out, ldo, M, N, K,
                              epilogue, workspace, device, on(stream));
}

int64_t cozyq_linear_workspace_bytes(int64_t M) {
    if (M < 0 || M > (int64_t{1} << 30)) return -1;
    return 4 * static_cast<int64_t>(cozyq::linear_workspace_ints(static_cast<int>(M)));
}

int cozyq_linear(int device, const void* x, int x_half, int rotation, int8_t* q, float* qs,
                 const int8_t* w, const float* w_scale, const void* bias, void* out, int64_t ldo,
                 int out_half, int M, int N, int K, int epilogue, int* workspace, void* stream) {
    return linear_checked(device, x, x_half, rotation, q, qs, w, w_scale, bias, out, ldo, out_half,
                          M, N, K, epilogue, workspace, false, stream);
}

int cozyq_linear_noalloc_max_rows(void) { return cozyq::linear_noalloc_max_rows(); }

static int linear_status_checked(int device, int* workspace, void* stream) {
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    int status = 0;
    const hipError_t e = cozyq::linear_status(workspace, device, on(stream), &status);
    if (e != hipSuccess) return e;
    return status ? hipErrorLaunchTimeOut : hipSuccess;
}

int cozyq_linear_status(int device, int* workspace, void* stream) {
    if (workspace == nullptr) return hipErrorInvalidValue;
    return linear_status_checked(device, workspace, stream);
}

int cozyq_linear_noalloc_status(int device, void* stream) {
    return linear_status_checked(device, nullptr, stream);
}

void cozyq_linear_test_spin_limit(int limit) { cozyq::linear_set_spin_limit(limit); }

int cozyq_linear_noalloc(int device, const void* x, int x_half, int rotation, int8_t* q, float* qs,
                         const int8_t* w, const float* w_scale, const void* bias, void* out,
                         int64_t ldo, int out_half, int M, int N, int K, int epilogue, void* stream) {
    return linear_checked(device, x, x_half, rotation, q, qs, w, w_scale, bias, out, ldo, out_half,
                          M, N, K, epilogue, nullptr, true, stream);
}

int cozyq_gemm(int device, int family, int fp8, const void* q, const float* scales,
               const void* w, const float* w_scale, const void* bias, void* out, int64_t ldo,
               int out_half, int M, int N, int K, int config, cozyq_allocate_fn allocate,
               void* allocate_context, void* stream) {
    (void)allocate; (void)allocate_context;
    if (family != 0) return hipErrorInvalidValue;
    return gemm_checked(device, fp8, q, scales, w, w_scale, bias, out, ldo, out_half, M, N, K, 0,
                        fp8 ? 16 : 256, config, stream);
}

int cozyq_gemm_config(int fp8, int M, int N, int K) {
    if (M < 1 || N < 1 || K < 1) return -1;
    return cozyq::gemm_config(fp8 != 0, M, N, K);
}

int cozyq_gemm_ex(int device, int fp8, const void* q, const float* scales, const void* w,
                  const float* w_scale, const void* bias, void* out, int64_t ldo, int out_half,
                  int M, int N, int K, int epilogue, void* stream) {
    return gemm_checked(device, fp8, q, scales, w, w_scale, bias, out, ldo, out_half, M, N, K,
                        epilogue, 16, -1, stream);
}

int cozyq_gemm_i32(int device, const int8_t* q, const int8_t* w, int32_t* acc, int M, int N,
                   int K, void* stream) {
    if (M < 1 || N < 1 || N % 8 || !fits(K, 16)) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::gemm_int8_acc(q, w, acc, M, N, K, on(stream));
}

int cozyq_w4a8_gemm(int device, const int8_t* q, const float* scales, const uint8_t* w,
                    const uint8_t* s, const float* codebook, const float* w_scale, const void* bias,
                    void* out, int out_half, int M, int N, int K, int config, void* stream) {
    if (M < 1 || N < 8 || N % 8 || !fits(K, 256)) return hipErrorInvalidValue;
    // Configs 1..4 are the narrow tiles; 0 and 5 (the 256-row tiles) have no fused 4-bit form.
    if (config == 0 || config >= 5) return hipErrorNotSupported;
    if (!aligned16(q) || !aligned16(w) || (reinterpret_cast<uintptr_t>(out) & 7))
        return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::gemm_w4a8_narrow(q, scales, w, s, codebook, w_scale, bias, out, out_half, M, N,
                                   K, config < 0 ? -1 : config, on(stream));
}

int cozyq_w4a8_unpack(int device, const uint8_t* w, const uint8_t* s, const float* codebook,
                      int8_t* out, int N, int K, void* stream) {
    if (N < 1 || !fits(K, 256)) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(w) & 7) || !aligned16(out)) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::w4a8_unpack(w, s, codebook, out, N, K, on(stream));
}

int cozyq_fp8_linear(int device, const void* x, int x_half, const uint8_t* w,
                     const float* w_scale, const void* bias, void* out, int out_half, int M,
                     int N, int K, void* stream) {
    if (M < 0 || N < 1 || N % 8 || !fits(K, 16)) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    if (!aligned16(x) || !aligned16(w) || (reinterpret_cast<uintptr_t>(out) & 7))
        return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::fp8_linear_small(x, x_half, w, w_scale, bias, out, out_half, M, N, K,
                                   on(stream));
}

int cozyq_mx_quantize(int device, const void* x, int x_half, uint8_t* q, uint8_t* scales, int M,
                      int K, void* stream) {
    if (M < 0 || !fits(K, 32)) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::mx_quantize(x, x_half, q, scales, M, K, on(stream));
}

int cozyq_mx_gemm(int device, const uint8_t* q, const uint8_t* q_scales, const uint8_t* w,
                  const uint8_t* w_scales, const void* bias, void* out, int64_t ldo, int out_half,
                  int M, int N, int K, void* stream) {
    if (M < 1 || N < 1 || N % 8 || !fits(K, 128)) return hipErrorInvalidValue;
    if (ldo < N || ldo % 8 || !aligned16(out)) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::gemm_mx(q, q_scales, w, w_scales, bias, out, ldo, out_half, M, N, K,
                          on(stream));
}

int cozyq_svdq_int4_quantize(int device, const void* x, int x_half, const float* p,
                             const void* down, uint8_t* act, uint16_t* ascales, void* la, int M,
                             int K, int R, void* stream) {
    if (M < 0 || !fits(K, 64) || (R != 16 && R != 32 && R != 64)) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    if (!aligned16(x) || !aligned16(p) || !aligned16(down) || !aligned16(act))
        return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::svdq_int4_quantize(x, x_half, p, down, act, ascales, la, M, K, R, on(stream));
}

int cozyq_svdq_int4_gemm(int device, const uint8_t* act, const uint16_t* ascales,
                         const uint8_t* w, const uint16_t* wscales, const void* la,
                         const void* up, const void* bias, void* out, int out_half, int M, int N,
                         int K, int R, void* stream) {
    if (M < 1 || N < 1 || N % 8 || !fits(K, 64) || (R != 16 && R != 32 && R != 64))
        return hipErrorInvalidValue;
    if (!aligned16(act) || !aligned16(w) || !aligned16(la) || !aligned16(up) || !aligned16(out) ||
        (reinterpret_cast<uintptr_t>(bias) & 3))
        return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::svdq_int4_gemm(act, ascales, w, wscales, la, up, bias, out, out_half, M, N, K,
                                 R, on(stream));
}

int cozyq_svdq_rows(int M) { return M < 0 ? -1 : cozyq::svdq_nvfp4_padded_rows(M); }

int cozyq_svdq_input_scale(int device, const void* x, int x_half, const float* p, int M, int K,
                           float* g, void* stream) {
    if (M < 0 || !fits(K, 64) || !g || !aligned16(x) || !aligned16(p)) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::svdq_nvfp4_input_scale(x, x_half != 0, p, M, K, g, on(stream));
}

static bool svdq_rank(int R) { return R == 32 || R == 64 || R == 128; }

int cozyq_svdq_quantize(int device, const void* x, int x_half, const float* p, const float* g,
                        const void* down, void* act, void* ascales, void* la, int M, int K, int R,
                        void* stream) {
    if (M < 0 || !fits(K, 64) || !svdq_rank(R)) return hipErrorInvalidValue;
    if (M > 0 && (!g || !aligned16(x) || !aligned16(p) || !aligned16(down) || !aligned16(act) ||
                  !aligned16(ascales) || !aligned16(la)))
        return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::svdq_nvfp4_quantize(x, x_half != 0, p, g, down, static_cast<uint8_t*>(act),
                                      static_cast<uint8_t*>(ascales), la, M, K, R, on(stream));
}

int cozyq_svdq_gemm(int device, const void* act, const void* ascales, const void* w,
                    const void* wscales, const float* gx, const float* gw, const float* c,
                    const void* la, const void* up, const void* bias, void* out, int out_half,
                    int M, int N, int K, int R, void* stream) {
    if (M < 1 || N < 8 || N % 8 || !fits(K, 64) || !svdq_rank(R) || !gx || !gw)
        return hipErrorInvalidValue;
    if (!aligned16(act) || !aligned16(ascales) || !aligned16(w) || !aligned16(wscales) ||
        !aligned16(la) || !aligned16(up) || !aligned16(out) || !aligned16(c) || !aligned16(bias))
        return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::svdq_nvfp4_gemm(static_cast<const uint8_t*>(act), static_cast<const uint8_t*>(ascales),
                                  static_cast<const uint8_t*>(w), static_cast<const uint8_t*>(wscales),
                                  gx, gw, c, la, up, bias, out, out_half != 0, M, N, K, R, on(stream));
}

int cozyq_decode(int device, int code, const void* w, const void* scale, int scale_type, int grid,
                 int block, int tiled, const float* scale_2, int scale_2_step, int second,
                 const void* post, int post_type, int post_mode, int high_first, void* out,
                 int out_type, int64_t rows, int64_t cols, int matrices, void* stream) {
    using namespace cozyq;
    if (code < kCodeI8 || code > kCodeE2m1 || scale_type < kNumF32 || scale_type > kNumE4m3 ||
        out_type < kNumF32 || out_type > kNumF16 || grid < kGridTensor || grid > kGridBlocks ||
        second < kSecondNone || second > kSecondDivide || post_mode < kPostNone ||
        post_mode > kPostColumn || rows < 0 || cols < 1 || matrices < 1 || matrices > 65535)
        return hipErrorInvalidValue;
    if (grid == kGridBlocks && block < 1) return hipErrorInvalidValue;
    if (tiled && grid != kGridBlocks) return hipErrorInvalidValue;
    if (code == kCodeE2m1 && cols % 2) return hipErrorInvalidValue;
    if ((second && !scale_2) || (post_mode && (!post || post_type > kNumE4m3 || post_type < 0)) ||
        !w || !scale || !out)
        return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    TableDecode a{};
    a.weight = static_cast<const uint8_t*>(w);
    a.weight_stride = code == kCodeE2m1 ? rows * cols / 2 : rows * cols;
    a.scale = scale;
    a.scale_type = scale_type;
    a.scale_size = scale_type <= kNumF16 ? (scale_type == kNumF32 ? 4 : 2) : 1;
    a.grid = grid;
    a.block = block;
    a.tiled = tiled;
    if (grid == kGridRow) {
        a.scale_stride = rows;
    } else if (grid == kGridBlocks) {
        const int64_t width = (cols + block - 1) / block;
        a.scale_stride = tiled ? ((rows + 127) / 128 * 128) * ((width + 3) / 4 * 4) : rows * width;
    }
    a.scale_2 = scale_2;
    a.scale_2_step = scale_2_step ? 1 : 0;
    a.second = second;
    a.post = post;
    a.post_type = post_type;
    a.post_mode = post_mode;
    a.high_first = high_first ? 1 : 0;
    a.out = out;
    a.out_stride = rows * cols;
    a.rows = rows;
    a.cols = cols;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return decode_table(a, code, out_type, matrices, on(stream));
}

int cozyq_decode_convrot(int device, const int8_t* w, const void* scale, int scale_type,
                         int rotation_size, void* out, int out_type, int64_t rows, int64_t cols,
                         void* stream) {
    using namespace cozyq;
    int digits = 0;
    for (int size = 4; size <= 65536; size *= 4) {
        ++digits;
        if (size == rotation_size) break;
    }
    if (rotation_size < 4 || rotation_size > 65536 || (1 << (2 * digits)) != rotation_size)
        return hipErrorInvalidValue;
    if (scale_type < kNumF32 || scale_type > kNumF16 || out_type < kNumF32 ||
        out_type > kNumF16 || rows < 0 || cols < 1 || cols % rotation_size || !w || !scale || !out)
        return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    // Groups of 64 and more are read and written 64 elements a lane, 16 bytes at a time.
    if (rotation_size >= 64 && (!aligned16(w) || !aligned16(out))) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return decode_convrot(w, scale, scale_type, out, out_type, rows, cols, digits, on(stream));
}

int cozyq_decode_svdq(int device, const uint8_t* w, const uint8_t* scale, int tiled,
                      int high_first, const float* scale_2, int divide, const void* channel_scale,
                      int channel_type, const void* smooth, int smooth_type, const void* down,
                      int down_type, const void* up, int up_type, int rank, void* out,
                      int out_type, int64_t rows, int64_t cols, void* stream) {
    using namespace cozyq;
    const auto plain = [](int t) { return t >= kNumF32 && t <= kNumF16; };
    if (rows < 0 || cols < 16 || cols % 16 || rank < 1 || !plain(smooth_type) ||
        !plain(down_type) || !plain(up_type) || !plain(out_type) ||
        (channel_scale && channel_type != kNumF32 && channel_type != kNumE4m3) || !w || !scale ||
        !scale_2 || !smooth || !down || !up || !out)
        return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    SvdqDecode a{};
    a.weight = w;
    a.scale = scale;
    a.tiled = tiled ? 1 : 0;
    a.high_first = high_first ? 1 : 0;
    a.divide = divide ? 1 : 0;
    a.scale_2 = scale_2;
    a.channel = channel_scale;
    a.channel_type = channel_type;
    a.smooth = smooth;
    a.smooth_type = smooth_type;
    a.down = down;
    a.down_type = down_type;
    a.up = up;
    a.up_type = up_type;
    a.rank = rank;
    a.out = out;
    a.rows = rows;
    a.cols = cols;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return decode_svdq(a, out_type, on(stream));
}

int cozyq_nvfp4_gemv(int device, const void* x, int x_half, const uint8_t* w, const uint8_t* scale,
                     const float* scale_2, void* out, int out_half, int M, int N, int K, void* stream) {
    if (M < 0 || M > 64 || N < 1 || K < 32 || K % 32 || K > cozyq::kMaxK || !w || !scale || !scale_2)
        return hipErrorInvalidValue;
    if (static_cast<int64_t>(N) * (K / 2) >= 0x7fffffff ||
        static_cast<int64_t>((N + 127) / 128 * 128) * ((K / 16 + 3) / 4 * 4) >= 0x7fffffff)
        return hipErrorNotSupported;
    if (M == 0) return hipSuccess;  // an empty x may have no address
    if (!x || !out || !aligned16(x) || (reinterpret_cast<uintptr_t>(w) & 3) || (reinterpret_cast<uintptr_t>(out) & 1))
        return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::nvfp4_gemv(x, x_half != 0, w, scale, scale_2, out, out_half != 0, M, N, K, on(stream));
}

int cozyq_nvfp4_gemm(int device, const void* x, int x_half, const uint8_t* w, const uint8_t* scale,
                     const float* scale_2, const void* bias, void* out, int out_half, int M, int N, int K,
                     void* stream) {
    if (M < 0 || N < 8 || N % 8 || !fits(K, 64) || !w || !scale || !scale_2) return hipErrorInvalidValue;
    if (static_cast<int64_t>(N) * (K / 2) >= 0x7fffffff ||
        static_cast<int64_t>((N + 127) / 128 * 128) * (K / 16) >= 0x7fffffff)
        return hipErrorNotSupported;
    if (M == 0) return hipSuccess;  // an empty x may have no address
    if (!x || !out || !aligned16(x) || !aligned16(w) || !aligned16(scale) || !aligned16(out) || !aligned16(bias))
        return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::nvfp4_gemm(x, x_half != 0, w, scale, scale_2, bias, out, out_half != 0, M, N, K, on(stream));
}

int cozyq_encode_int8_convrot(int device, const void* w, int w_type, int8_t* q, float* scale,
                               int64_t rows, int K, void* stream) {
    if (w_type < 0 || w_type > 2 || rows < 0 || rows > 0x7fffffff || !fits(K, 256)) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    if (!aligned16(w) || !aligned16(q)) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::encode_rotated(w, w_type, rows, K, q, scale, nullptr, nullptr, nullptr, false, on(stream));
}

int cozyq_encode_w4a8(int device, const void* w, int w_type, const float* codebook, uint8_t* codes,
                      uint8_t* group_scale, float* scale, int64_t rows, int K, void* stream) {
    if (w_type < 0 || w_type > 2 || rows < 0 || rows > 0x7fffffff || !fits(K, 256) || !codebook)
        return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    if (!aligned16(w) || (reinterpret_cast<uintptr_t>(codes) & 7)) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::encode_rotated(w, w_type, rows, K, nullptr, scale, codes, group_scale, codebook, true,
                                 on(stream));
}

int cozyq_encode_fp8_rowwise(int device, const void* w, int w_type, uint8_t* q, float* scale,
                             int64_t rows, int K, void* stream) {
    if (w_type < 0 || w_type > 2 || rows < 0 || rows > 0x7fffffff || !fits(K, 8)) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    if (!aligned16(w) || (reinterpret_cast<uintptr_t>(q) & 7)) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::encode_fp8_rowwise(w, w_type, rows, K, q, scale, on(stream));
}

int cozyq_encode_mxfp8(int device, const void* w, int w_type, uint8_t* q, uint8_t* scale, int tiled,
                       int64_t rows, int K, void* stream) {
    if (w_type < 0 || w_type > 2 || rows < 0 || !fits(K, 32)) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    if (!aligned16(w) || (reinterpret_cast<uintptr_t>(q) & 7)) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::encode_mx(w, w_type, rows, K, q, scale, tiled ? 1 : 0, on(stream));
}

int cozyq_encode_nvfp4(int device, const void* w, int w_type, uint8_t* codes, uint8_t* scale,
                       float* scale_2, uint32_t* amax, unsigned long long* saturated, int64_t rows,
                       int K, void* stream) {
    if (w_type < 0 || w_type > 2 || rows < 0 || !fits(K, 16) || !amax || !saturated || !scale_2)
        return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    if (!aligned16(w) || (reinterpret_cast<uintptr_t>(codes) & 7)) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::encode_nvfp4(w, w_type, rows, K, amax, codes, scale, scale_2, saturated, on(stream));
}

int cozyq_encode_svdq_int4(int device, const void* w, int w_type, const float* p, const void* down,
                           const void* up, int rank, uint8_t* codes, uint16_t* scales, int64_t rows,
                           int K, void* stream) {
    if (rows < 0 || rank < 0 || rank > 1024 || w_type < 0 || w_type > 2 || !fits(K, 64))
        return hipErrorInvalidValue;
    if (rows > 0 && (!w || !p || !codes || !scales || (rank > 0 && (!down || !up)) ||
                     !aligned16(w) || !aligned16(down) || !aligned16(codes) || !aligned16(scales)))
        return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::encode_svdq_int4(w, w_type, p, down, up, rank, rows, K, codes, scales, on(stream));
}

int cozyq_measure(int device, const void* w, int w_type, const float* decoded, int64_t total,
                  double* partial, int parts, double* out, void* stream) {
    if (w_type < 0 || w_type > 2 || total < 0 || parts < 1 || !w || !decoded || !partial || !out)
        return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::measure(w, w_type, decoded, total, partial, parts, out, on(stream));
}

int cozyq_bake_rotate_factor(int device, const float* down, float* out, int64_t rank, int64_t cols,
                             void* stream) {
    if (rank < 0 || cols < 0 || cols % 256 || rank * cols > (int64_t{1} << 40)) return hipErrorInvalidValue;
    if (rank == 0 || cols == 0) return hipSuccess;
    if (!down || !out) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::rotate_factor(down, out, rank * cols / 256, on(stream));
}

// Tiles are 64 rows × 128 columns: the grid's y extent bounds the rows.
static bool bake_shape(int64_t rows, int64_t cols, int64_t rank) {
    return rows >= 0 && cols >= 0 && rank >= 0 && rows <= 65535LL * 64 && cols <= 0x7fffffff &&
           rank <= 0x7fffffff && rows * cols <= (int64_t{1} << 40);
}

// A bake's options: gain only for plain and nvfp4 rows (a row-scaled weight takes it in its
// scale), known flags only.
static bool bake_options(int form, const float* gain, int flags) {
    if (flags & ~(cozyq::kBakeNearest | cozyq::kBakeNoDelta)) return false;
    return !gain || form <= cozyq::kBakeF32 || form == cozyq::kBakeNvfp4;
}

int cozyq_bake(int device, int form, void* data, const float* scale, const float* up, const float* down,
               const float* gain, const float* more, const float* rescale, int64_t rows, int64_t cols,
               int64_t rank, uint32_t seed, int flags, void* stream) {
    if (form < cozyq::kBakeBf16 || form > cozyq::kBakeInt8 || !bake_shape(rows, cols, rank) ||
        !bake_options(form, gain, flags) || (rescale && (form != cozyq::kBakeRowwise || (flags & cozyq::kBakeNoDelta))))
        return hipErrorInvalidValue;
    if (rows == 0 || cols == 0) return hipSuccess;
    const bool scaled = form == cozyq::kBakeRowwise || form == cozyq::kBakeInt8;
    if (!data || (scaled && !scale) || (rank > 0 && (!up || !down))) return hipErrorInvalidValue;
    const size_t size = form == cozyq::kBakeF32 ? 4 : (form <= cozyq::kBakeF16 ? 2 : 1);
    if (reinterpret_cast<uintptr_t>(data) % size) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::bake(form, data, scale, up, down, cozyq::BakeOptions{gain, more, flags, rescale}, static_cast<int>(rows),
                       static_cast<int>(cols), static_cast<int>(rank), seed, on(stream));
}

int cozyq_bake_nvfp4(int device, uint8_t* data, uint8_t* blocks, const float* second, const float* up,
                     const float* down, const float* gain, const float* more, int64_t rows, int64_t cols,
                     int64_t rank, uint32_t seed, int flags, void* stream) {
    if (!bake_shape(rows, cols, rank) || cols % 16 || !bake_options(cozyq::kBakeNvfp4, gain, flags))
        return hipErrorInvalidValue;
    if (rows == 0 || cols == 0) return hipSuccess;
    if (!data || !blocks || !second || (rank > 0 && (!up || !down))) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::bake_nvfp4(data, blocks, second, up, down, cozyq::BakeOptions{gain, more, flags, nullptr},
                             static_cast<int>(rows), static_cast<int>(cols), static_cast<int>(rank), seed, on(stream));
}

int cozyq_bake_nvfp4_refit(int device, uint8_t* data, uint8_t* blocks, const float* second, double level,
                           const float* up, const float* down, const float* gain, const float* more, int64_t rows,
                           int64_t cols, int64_t rank, uint32_t seed, int flags, void* stream) {
    if (!bake_shape(rows, cols, rank) || cols % 16 || (flags & ~cozyq::kBakeNearest) || !(level > 0.0) ||
        !(level < 3.4e38))
        return hipErrorInvalidValue;
    if (rows == 0 || cols == 0) return hipSuccess;
    if (!data || !blocks || !second || (rank > 0 && (!up || !down))) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    cozyq::BakeOptions o{gain, more, flags, nullptr};
    o.refit = true;
    o.level = level;
    return cozyq::bake_nvfp4(data, blocks, second, up, down, o, static_cast<int>(rows), static_cast<int>(cols),
                             static_cast<int>(rank), seed, on(stream));
}

static int bake_rows(int device, int form, const void* data, const float* scale, const uint8_t* blocks,
                     const float* second, const float* up, const float* down, const float* gain,
                     const float* more, int64_t rows, int64_t cols, int64_t rank, float* out, bool amax,
                     void* stream) {
    if (form < cozyq::kBakeBf16 || form > cozyq::kBakeNvfp4 || !bake_shape(rows, cols, rank) ||
        (form == cozyq::kBakeNvfp4 && cols % 16))
        return hipErrorInvalidValue;
    // A gain multiplies plain and nvfp4 rows only (the row-scaled forms take none).
    if (gain && (form == cozyq::kBakeRowwise || form == cozyq::kBakeInt8)) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    const bool scaled = form == cozyq::kBakeRowwise || form == cozyq::kBakeInt8;
    if (!out || (cols > 0 && !data) || (scaled && !scale) || (form == cozyq::kBakeNvfp4 && (!blocks || !second)) ||
        (rank > 0 && cols > 0 && (!up || !down)))
        return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::bake_norms(form, data, scale, blocks, second, up, down, gain, more, static_cast<int>(rows),
                             static_cast<int>(cols), static_cast<int>(rank), out, amax, on(stream));
}

int cozyq_bake_norms(int device, int form, const void* data, const float* scale, const uint8_t* blocks,
                     const float* second, const float* up, const float* down, int64_t rows, int64_t cols,
                     int64_t rank, float* out, void* stream) {
    return bake_rows(device, form, data, scale, blocks, second, up, down, nullptr, nullptr, rows, cols, rank, out,
                     false, stream);
}

int cozyq_bake_row_amax(int device, int form, const void* data, const float* scale, const uint8_t* blocks,
                        const float* second, const float* up, const float* down, const float* gain,
                        const float* more, int64_t rows, int64_t cols, int64_t rank, float* out, void* stream) {
    return bake_rows(device, form, data, scale, blocks, second, up, down, gain, more, rows, cols, rank, out, true,
                     stream);
}

int cozyq_bake_feedback(int device, uint8_t* data, const float* scale, const float* fresh, const float* up,
                        const float* down, const float* more, int64_t rows, int64_t cols, int64_t rank,
                        void* stream) {
    if (!bake_shape(rows, cols, rank)) return hipErrorInvalidValue;
    if (rows == 0 || cols == 0) return hipSuccess;
    if (!data || !scale || !fresh || (rank > 0 && (!up || !down))) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::bake_feedback(data, scale, fresh, up, down, more, static_cast<int>(rows), static_cast<int>(cols),
                                static_cast<int>(rank), on(stream));
}

int cozyq_bake_stats(int device, int form, const void* before, const void* after, const float* scale_before,
                     const float* scale_after, const uint8_t* blocks_before, const uint8_t* blocks_after,
                     const float* second, const float* second_after, const float* gain, const float* more,
                     const float* up, const float* down, int64_t rows, int64_t cols, int64_t rank, double* partial,
                     void* stream) {
    if (form < cozyq::kBakeBf16 || form > cozyq::kBakeNvfp4 || !bake_shape(rows, cols, rank) ||
        (form == cozyq::kBakeNvfp4 && cols % 16))
        return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    const bool scaled = form == cozyq::kBakeRowwise || form == cozyq::kBakeInt8;
    if (!partial || (cols > 0 && (!before || !after)) || (scaled && (!scale_before || !scale_after)) ||
        (form == cozyq::kBakeNvfp4 && (!blocks_before || !blocks_after || !second)) ||
        (rank > 0 && cols > 0 && (!up || !down)))
        return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    const cozyq::BakeStats st{before, after, scale_before, scale_after, blocks_before, blocks_after, second, gain, more,
                              second_after};
    return cozyq::bake_stats(form, st, up, down, static_cast<int>(rows), static_cast<int>(cols),
                             static_cast<int>(rank), partial, on(stream));
}

void cozyq_host_e4m3(const float* in, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = cozyq::e4m3_rn(in[i]);
}

int cozyq_probe_e4m3(int device, const float* in, uint8_t* out, int64_t n, void* stream) {
    if (n < 0 || n % 2) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::e4m3_probe(in, out, n, on(stream));
}

int cozyq_probe_e2m1(int device, const float* in, uint8_t* out, int64_t n, void* stream) {
    if (n < 0 || n % 2) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::e2m1_probe(in, out, n, on(stream));
}

int cozyq_probe_div(int device, const float* x, const float* s, float* out, int64_t n,
                    void* stream) {
    if (n < 0) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::div_probe(x, s, out, n, on(stream));
}

void cozyq_host_mx_byte(const float* amax, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = cozyq::mx_byte(amax[i]);
}

int cozyq_probe_mfma(int device, int kind, const void* a, const void* b, const void* sa,
                     const void* sb, void* d, void* stream) {
    if (kind < 0 || kind > 8) return hipErrorInvalidValue;
    const OnDevice guard(device);
    if (guard.error() != hipSuccess) return guard.error();
    return cozyq::mfma_probe(kind, a, b, sa, sb, d, on(stream));
}

}  // extern "C"
