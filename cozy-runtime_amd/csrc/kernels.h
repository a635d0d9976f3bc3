// Launchers of the gfx950 kernels, called by the C ABI (abi.hip) after it has checked the
// arguments. Each enqueues on `s` and returns the launch's error code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cozyq {

// The producer's prologue folded into the quantize pass (reference: kernels/csrc/gemm/int8.h:
// 25-47): activation(norm(x) · (1 + scale) + shift). Tables are in x's dtype, rows
// `*_stride` elements apart; row r of x reads table row r / rows_per_entry. norm 0 none, 1
// layer, 2 RMS (no affine); act 0 none, 1 GELU (erf), 2 tanh-GELU, 3 SiTU on [hidden | gate]
// rows of 2K, 4 SwiGLU (gate rows in x and up rows in `up`; without `up`, [up | gate] rows).
struct Prologue {
    const uint16_t* scale;
    const uint16_t* shift;
    int64_t scale_stride, shift_stride;
    int rows_per_entry, norm;
    float eps;
    int act;
    const uint16_t* up;
};

// `pro` may be null (no prologue); with one, rotation must be 256.
hipError_t rotate_quantize(const void* x, bool x_half, int8_t* q, float* scales, int M, int K,
                           int rotation, const Prologue* pro, hipStream_t s);
hipError_t fp8_quantize(const void* x, bool x_half, uint8_t* q, float* scales, int M, int K,
                        const Prologue* pro, hipStream_t s);
hipError_t mx_quantize(const void* x, bool x_half, uint8_t* q, uint8_t* scales, int M, int K,
                       hipStream_t s);

// The fused int8 linear (linear.hip): x's rows rotated (256, 128 or 0) and quantized per token
// into q / qs, then the 256x256-tile int8 GEMM with its epilogue, in one persistent launch; out
// in x's dtype. K <= 4096. `work` holds linear_workspace_ints(M) int32 counters, zero before the
// first launch and zero again after each.
int linear_workspace_ints(int M);
hipError_t linear_int8(const void* x, bool half, int rotation, int8_t* q, float* qs, const int8_t* w,
                       const float* ws, const void* bias, void* out, int64_t ldo, int M, int N, int K,
                       int epilogue, int* work, int device, hipStream_t s);
// linear_int8 with its counters in the library's own device array (no workspace, no
// allocation): M <= linear_noalloc_max_rows(), else hipErrorInvalidValue. Calls that overlap on
// one GPU race on the array.
int linear_noalloc_max_rows();
// The status word of a fused linear's counters (`work`, or the allocation-free array when null):
// 1 if a launch since the last read gave up waiting for its rows (its tiles were written as NaN),
// else 0; reading it synchronizes `s` and clears the word.
hipError_t linear_status(int* work, int device, hipStream_t s, int* status);
// Test hook: the spin limit of later fused launches (0 the default; negative: every wait gives
// up at once).
void linear_set_spin_limit(int limit);
hipError_t linear_int8_noalloc(const void* x, bool half, int rotation, int8_t* q, float* qs,
                               const int8_t* w, const float* ws, const void* bias, void* out,
                               int64_t ldo, int M, int N, int K, int epilogue, int device,
                               hipStream_t s);

// The rowwise GEMMs' tile configs: 0 the 256x256 kernel, 1..4 the narrow kernels' 128x128,
// 128x64, 64x64 and 32x64, 5 the 256x192 kernel (kGemmConfigs in all); -1 lets gemm_config
// choose by shape. Every config gives the same int8 output bit for bit; an unknown config is
// hipErrorNotSupported.
constexpr int kGemmConfigs = 6;
int gemm_config(bool fp8, int M, int N, int K);
// Whether 256x192 tiles fill the 256 CUs in fewer rounds than 256x256 ones at this shape (the
// large-tile choice of gemm_config, the MX GEMM and the svdq.nvfp4 GEMM).
bool wide_tile(int M, int N);
int narrow_config(int M, int N);
hipError_t gemm_int8(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                     const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                     int epilogue, int config, hipStream_t s);
hipError_t gemm_fp8(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                    const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                    int epilogue, int config, hipStream_t s);
hipError_t gemm_mx(const uint8_t* q, const uint8_t* qe, const uint8_t* w, const uint8_t* we,
                   const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                   hipStream_t s);
hipError_t gemm_int8_acc(const int8_t* q, const int8_t* w, int32_t* acc, int M, int N, int K,
                         hipStream_t s);

hipError_t gemm_fp8_narrow(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                           const void* bias, void* out, int64_t ldo, bool out_half, int M, int N,
                           int K, int epilogue, int config, hipStream_t s);

// w4a8.convrot: codes [N, K/2], E4M3 group scales [N, K/16], codebook (16 float32 levels or
// null for q − 8); the fused narrow-tile GEMM (int8 q [M, K], the int8 epilogue, out [M, N]) and
// the unpack to int8 levels [N, K]. The fused GEMM takes configs 1..4 (-1: narrow_config).
hipError_t gemm_w4a8_narrow(const int8_t* q, const float* xs, const uint8_t* codes,
                            const uint8_t* group_scale, const float* codebook, const float* ws,
                            const void* bias, void* out, bool out_half, int M, int N, int K,
                            int config, hipStream_t s);
hipError_t w4a8_unpack(const uint8_t* codes, const uint8_t* group_scale, const float* codebook,
                       int8_t* out, int N, int K, hipStream_t s);
hipError_t gemm_int8_narrow(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                            const void* bias, void* out, int64_t ldo, bool out_half, int M, int N,
                            int K, int epilogue, int config, hipStream_t s);
// The int8 product on a 16-row weight tile a workgroup for 1..32 quantized rows, K <= 4096,
// N % 8 == 0 (hipErrorNotSupported elsewhere); the same bits as every tile config.
hipError_t int8_rows_gemm(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                          const void* bias, void* out, int64_t ldo, bool out_half, int M, int N,
                          int K, hipStream_t s);

// The compute units of `device` (256 on MI355X), read once per device.
int cu_count(int device);

// The fused int8 linear for 1..4 rows (rotate H256 + quantize + GEMV in one launch);
// hipErrorNotSupported past int8_gemv_max_k(M).
// The widest rows the fused few-row int8 linear takes at M rows (0 past 4): 32768 at M = 1,
// 16384 at 2, 12288 at 3 and 4.
int int8_gemv_max_k(int M);
hipError_t int8_linear_small(const void* x, bool x_half, const int8_t* w, const float* ws,
                             const void* bias, void* out, bool out_half, int M, int N, int K,
                             hipStream_t s);
// The int8 GEMV on quantized rows (cozyq_gemm's int8 product, 1..4 rows): K <= 32768 at 1 row,
// 16384 at 2, 12288 at 3..4, N % 4 == 0; hipErrorNotSupported elsewhere. The same bits as every
// tile.
hipError_t int8_codes_gemv(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                           const void* bias, void* out, int64_t ldo, bool out_half, int M, int N,
                           int K, hipStream_t s);
// The fused fp8 linear for 1..4 rows (the GEMV, M·K <= 16384) and 5..16 rows (K <= 4096);
// hipErrorNotSupported elsewhere.
hipError_t fp8_linear_small(const void* x, bool x_half, const uint8_t* w, const float* ws,
                            const void* bias, void* out, bool out_half, int M, int N, int K,
                            hipStream_t s);

hipError_t svdq_int4_quantize(const void* x, bool x_half, const float* p, const void* down,
                              uint8_t* act, uint16_t* ascales, void* la, int M, int K, int R,
                              hipStream_t s);
hipError_t svdq_int4_gemm(const uint8_t* act, const uint16_t* ascales, const uint8_t* w,
                          const uint16_t* wscales, const void* la, const void* up,
                          const void* bias, void* out, bool out_half, int M, int N, int K, int R,
                          hipStream_t s);

// ------------------------------------------------------------------ stored-format decode
// Element codes, numeric part dtypes, scale grids and second-level modes of the decode kernels
// (internal/encoding/formats.py:438-868; internal/decode_cores.py:196-230).
enum DecodeCode : int { kCodeI8 = 0, kCodeE4m3 = 1, kCodeE5m2 = 2, kCodeE2m1 = 3 };
enum DecodeNum : int { kNumF32 = 0, kNumBf16 = 1, kNumF16 = 2, kNumE8m0 = 3, kNumE4m3 = 4 };
enum DecodeGrid : int { kGridTensor = 0, kGridRow = 1, kGridCol = 2, kGridBlocks = 3 };
enum DecodeSecond : int { kSecondNone = 0, kSecondMultiply = 1, kSecondDivide = 2 };
enum DecodePost : int { kPostNone = 0, kPostOne = 1, kPostColumn = 2 };

// One matrix [rows, cols] (or a stack of them, `weight_stride` bytes, `scale_stride` scale
// elements and `out_stride` outputs apart; `scale_2_step` 1 for a factor per matrix).
struct TableDecode {
    const uint8_t* weight;
    int64_t weight_stride;
    const void* scale;
    int64_t scale_stride;
    int scale_type, scale_size, grid, block, tiled;
    const float* scale_2;
    int scale_2_step, second;
    const void* post;
    int post_type, post_mode, high_first;
    void* out;
    int64_t out_stride;
    int64_t rows, cols;
};

// svdq.nvfp4's W4A4 linear (svdq_nvfp4.hip): the activation's second level g_x from x and p;
// x -> the nvfp4 operand (act [Rows(M), K/2], ascales [Rows(M), K/16], la [Rows(M), R], Rows(M)
// = svdq_nvfp4_padded_rows(M), rows past M zero); the GEMM out [M, N] = (A·Wᵀ)·gx·gw·c + la·upᵀ
// + bias, one rounding (c and bias may be null). K % 64 == 0, R in {32, 64, 128}, N % 8 == 0.
int svdq_nvfp4_padded_rows(int M);
hipError_t svdq_nvfp4_input_scale(const void* x, bool x_half, const float* p, int M, int K,
                                  float* g, hipStream_t s);
hipError_t svdq_nvfp4_quantize(const void* x, bool x_half, const float* p, const float* g,
                               const void* down, uint8_t* act, uint8_t* ascales, void* la, int M,
                               int K, int R, hipStream_t s);
hipError_t svdq_nvfp4_gemm(const uint8_t* act, const uint8_t* ascales, const uint8_t* w,
                           const uint8_t* wscales, const float* gx, const float* gw,
                           const float* c, const void* la, const void* up, const void* bias,
                           void* out, bool out_half, int M, int N, int K, int R, hipStream_t s);

// svdq.nvfp4: codes [rows, cols/2], E4M3 scales per 16 (row-major or 128x4 tiles), scale_2,
// optional channel scale [rows], smoothing [cols], lowrank_down [rank, cols], lowrank_up
// [rows, rank].
struct SvdqDecode {
    const uint8_t* weight;
    const uint8_t* scale;
    int tiled, high_first, divide;
    const float* scale_2;
    const void* channel;
    int channel_type;
    const void* smooth;
    int smooth_type;
    const void* down;
    int down_type;
    const void* up;
    int up_type, rank;
    void* out;
    int64_t rows, cols;
};

hipError_t decode_table(const TableDecode& a, int code, int out_type, int matrices, hipStream_t s);
// `digits` = k of the 4^k group; groups of 64 and more need total % 64 == 0 and 16-byte
// aligned parts (hipErrorInvalidValue otherwise).
hipError_t decode_convrot(const int8_t* w, const void* scale, int scale_type, void* out, int out_type,
                          int64_t rows, int64_t cols, int digits, hipStream_t s);
hipError_t decode_svdq(const SvdqDecode& a, int out_type, hipStream_t s);

// nvfp4 W4A16 GEMV (nvfp4.hip): out [M, N] = round((x [M, K] · decode(w)ᵀ) · scale_2), M ≤ 64,
// codes [N, K/2] low nibble first, E4M3 scales in cuBLAS's 128x4 tiles, K % 32 == 0.
hipError_t nvfp4_gemv(const void* x, bool x_half, const uint8_t* w, const uint8_t* scale, const float* scale_2,
                      void* out, bool out_half, int M, int N, int K, hipStream_t s);

// nvfp4 W4A16 GEMM (svdq_nvfp4.hip), 256x256 tiles: out [M, N] = round((x · decode(w)ᵀ) · scale_2
// + bias), W decoded exactly into x's dtype on the way to the MFMA; the same operands as
// nvfp4_gemv, K % 64 == 0, N % 8 == 0; bias [N] in out's dtype or null.
hipError_t nvfp4_gemm(const void* x, bool x_half, const uint8_t* w, const uint8_t* scale, const float* scale_2,
                      const void* bias, void* out, bool out_half, int M, int N, int K, hipStream_t s);

// Weight encoders (encode.hip), input float32 / bf16 / fp16 by `in_type` (kNumF32 .. kNumF16),
// row-major [rows, K]. encode_rotated: int8.convrot (q, scale) or, with w4, w4a8.convrot (codes
// [rows, K/2], group_scale [rows, K/16], scale) against a 16-entry codebook; K % 256 == 0.
// encode_nvfp4 needs a zeroed `amax` word and `saturated` counter.
hipError_t encode_rotated(const void* w, int in_type, int64_t rows, int K, int8_t* q, float* scale, uint8_t* codes,
                          uint8_t* group_scale, const float* codebook, bool w4, hipStream_t s);
hipError_t encode_fp8_rowwise(const void* w, int in_type, int64_t rows, int K, uint8_t* q, float* scale,
                              hipStream_t s);
hipError_t encode_mx(const void* w, int in_type, int64_t rows, int K, uint8_t* q, uint8_t* scale, int tiled,
                     hipStream_t s);
hipError_t encode_nvfp4(const void* w, int in_type, int64_t rows, int K, uint32_t* amax, uint8_t* codes,
                        uint8_t* scale, float* scale_2, unsigned long long* saturated, hipStream_t s);
// svdq.int4g64: codes [rows, K/2] and fp16 group scales [rows, K/64] of (w − up·down) / p, up
// [rows, rank] and down [rank, K] bf16, p [K] f32; K % 64 == 0.
hipError_t encode_svdq_int4(const void* w, int in_type, const float* p, const void* down,
                            const void* up, int rank, int64_t rows, int K, uint8_t* codes,
                            uint16_t* scales, hipStream_t s);
// [Σ(w − d)², Σ w², max |w − d|] in float64 into `out`, through `parts` float64 triples.
hipError_t measure(const void* w, int in_type, const float* d, int64_t total, double* partial, int parts,
                   double* out, hipStream_t s);

// LoRA bake (bake.hip), in place: the stored forms of the reference's fused bake
// (internal/lora_bake.py:768); nvfp4 has its own entry.
enum BakeForm { kBakeBf16 = 0, kBakeF16 = 1, kBakeF32 = 2, kBakeRowwise = 3, kBakeInt8 = 4, kBakeNvfp4 = 5 };
// kBakeNearest: round to nearest (ties to even) instead of stochastically; kBakeNoDelta: the
// rows times their gain alone (`gain_rows`).
enum BakeFlags { kBakeNearest = 1, kBakeNoDelta = 2 };
// Beyond the fused law: a float32 gain per row (plain and nvfp4 rows), dense float32 rows
// [rows, cols] added to the delta, flags. All null / 0: the fused law exactly.
struct BakeOptions {
    const float* gain;
    const float* more;
    int flags;
    const float* rescale;  // kBakeRowwise: each row's new scale [rows] (`refit`, `regrid`); null keeps
    bool refit = false;    // kBakeNvfp4: every block refitted on the new second level `level`
    double level = 0.0;
};
// data [rows, cols] of the form, scale float32 [rows] (kBakeRowwise, kBakeInt8), up float32
// [rows, rank], down float32 [rank, cols] (kBakeInt8: already rotated), the 32-bit seed.
hipError_t bake(int form, void* data, const float* scale, const float* up, const float* down, const BakeOptions& o,
                int rows, int cols, int rank, uint32_t seed, hipStream_t s);
// codes [rows, cols/2], E4M3 block bytes [rows, cols/16], second level at `second`; cols % 16 == 0.
hipError_t bake_nvfp4(uint8_t* data, uint8_t* blocks, const float* second, const float* up, const float* down,
                      const BakeOptions& o, int rows, int cols, int rank, uint32_t seed, hipStream_t s);
// Row L2 norms (or, with `amax`, row maxima of |·|) of the decoded weight (times `gain`, float32
// [rows], if given) plus up @ down (plus `more` [rows, cols], if given) into out [rows] (float32);
// form as above, kBakeNvfp4 with `blocks` and `second`.
hipError_t bake_norms(int form, const void* data, const float* scale, const uint8_t* blocks, const float* second,
                      const float* up, const float* down, const float* gain, const float* more, int rows, int cols,
                      int rank, float* out, bool amax, hipStream_t s);
// fp8.rowwise with error feedback: codes from (e4m3·scale + delta) / fresh rounded to nearest
// with each run of 32 columns carrying its rounding error; fresh = the rows' scales after; `more`
// (dense rows [rows, cols], or null) adds to the delta.
hipError_t bake_feedback(uint8_t* data, const float* scale, const float* fresh, const float* up, const float* down,
                         const float* more, int rows, int cols, int rank, hipStream_t s);
// A bake's accounting: the weight before and after (each form's parts), the same gain and dense
// rows the bake took; partial receives 7 doubles per 64-row workgroup ([target², delta², error²,
// kept, saturated, effect, effect error]). rank ≤ 128.
struct BakeStats {
    const void* before;
    const void* after;
    const float* scale_before;
    const float* scale_after;
    const uint8_t* blocks_before;
    const uint8_t* blocks_after;
    const float* second;
    const float* gain;
    const float* more;
    const float* second_after = nullptr;  // nvfp4: the level `after` decodes at; null: `second`
};
hipError_t bake_stats(int form, const BakeStats& st, const float* up, const float* down, int rows, int cols, int rank,
                      double* partial, hipStream_t s);
// out = each 256-group of down times H256 / 16; `groups` = rank · cols / 256.
hipError_t rotate_factor(const float* down, float* out, int64_t groups, hipStream_t s);

}  // namespace cozyq

namespace cozyq {
hipError_t div_probe(const float* x, const float* s, float* out, int64_t n, hipStream_t st);
hipError_t e4m3_probe(const float* in, uint8_t* out, int64_t n, hipStream_t s);
hipError_t e2m1_probe(const float* in, uint8_t* out, int64_t n, hipStream_t s);
hipError_t mfma_probe(int kind, const void* a, const void* b, const void* sa, const void* sb,
                      void* d, hipStream_t s);
}  // namespace cozyq
