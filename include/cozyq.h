/* cozyq — MI355X (gfx950) quantized-linear kernels behind a C ABI.
 *
 * The drop-in replacement for cozy-runtime's native `_kernels._gemm` module
 * (reference: kernels/csrc/gemm.cpp:194-222, stubs src/cozy_runtime/_kernels/_gemm.pyi:1-116).
 * Arguments are raw device pointers, sizes and a HIP stream: neither torch nor Python is a
 * build input, and the caller allocates every operand and output. Every call returns a
 * hipError_t code: 0 ran; hipErrorNotSupported (cozyq_not_supported()) means no kernel takes
 * this shape and the caller decides; hipErrorInvalidValue rejects arguments; hipErrorOutOfMemory
 * (cozyq_out_of_memory()) is the device's. Launches go on `stream` with `device` current for the
 * call and the caller's device restored afterwards. No entry point allocates or synchronizes,
 * so each may be recorded into a HIP graph.
 *
 * Layouts: activations and outputs are row-major with the reduction axis K last; weights are
 * [N, K] row-major (the nn.Linear layout); per-row scales are float32. `x_half` / `out_half`
 * select fp16 (1) or bf16 (0) for 16-bit tensors.
 */
#ifndef COZYQ_H
#define COZYQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Constants (reference: gemm.cpp:194-203 `NOT_SUPPORTED`, `OUT_OF_MEMORY`, `GEMV_ROWS`, `MAX_K`). */
int cozyq_not_supported(void);
int cozyq_out_of_memory(void);
int cozyq_gemv_rows(void);
int cozyq_max_k(void);
/* The device-code target this library carries, e.g. "gfx950". */
const char* cozyq_arch(void);

/* hipGetErrorName of a returned code (reference: gemm.cpp:204 `error_name`). */
const char* cozyq_error_name(int code);

/* Per-token activation quantization (reference: gemm.cpp:83-115 `quantize`, law
 * internal/int8_linear.py:422-428 for int8 and internal/fp8_linear.py:56-63 for fp8).
 * fp8 = 0: each row rotated by H256/16 (regular H4⊗H4⊗H4⊗H4) and quantized to int8 with
 *          scales[m] = max(amax/127, 1e-12); K % 256 == 0.
 * fp8 = 1: each row quantized to OCP E4M3 with scales[m] = max(amax/448, 1e-12); K % 16 == 0.
 * q: [M, K] (int8 or e4m3 bytes); scales: [M] float32. K <= cozyq_max_k().
 * The producer's prologue (reference: int8.h:25-47, rotate.cu:195-282) is applied in float32
 * before the rotation / quantization: activation(norm(x) · (1 + scale[e]) + shift[e]) with
 * e = m / rows_per_entry. norm 0 none, 1 layer, 2 RMS (no affine; eps inside the rsqrt);
 * scale/shift: tables in x's dtype, rows scale_stride/shift_stride elements apart (multiples of
 * 8, 16-byte aligned), or NULL; activation 0 none, 1 GELU (erf), 2 tanh-GELU, 3 SiTU (x rows
 * are [hidden | gate], 2K wide: 4 tanh(g/4) sigmoid(g) · 25 tanh(h/25)), 4 SwiGLU (x holds the
 * gate rows and `up` the up rows, [M, K] each, silu(gate) · up with each product rounded to
 * x's dtype; without `up`, x rows are [up | gate], 2K wide). The gated activations (3, 4) take
 * no norm or tables; `up` only with 4. Violations return hipErrorInvalidValue. */
int cozyq_quantize(int device, int fp8, const void* x, int x_half, void* q, float* scales, int M,
                   int K, const void* scale, const void* shift, int64_t scale_stride,
                   int64_t shift_stride, int rows_per_entry, int norm, float eps, int activation,
                   const void* up, void* stream);

/* int8 quantization with an explicit rotation (no reference counterpart: the reference's int8
 * lane always rotates by 256). rotation 256 is cozyq_quantize's law; 0 is plain per-token int8
 * (K % 16 == 0); 128 is H2⊗H4⊗H4⊗H4 with the unnormalized sums quantized and the 1/sqrt(128)
 * folded into scales[m] (K % 128 == 0). */
int cozyq_quantize_rot(int device, const void* x, int x_half, int8_t* q, float* scales, int M,
                       int K, int rotation, void* stream);

/* The fused few-row int8 linear (reference: gemm.cpp:117-125 `gemv`, rotate.cu:351-407): each
 * row of x rotated and quantized by cozyq_quantize's int8 law inside the kernel, then
 * out = ((acc·s_x)·w_scale, cast) + bias in the output dtype, bit for bit the CPU law. Served for
 * 1 <= M <= 4 with K up to 32768 (M = 1), 16384 (M = 2) or 12288 (M = 3, 4) — the reference's
 * range, M·K + M·(warps + 1)·4 <= 48 KiB, and more at M = 2 — N % 8 == 0, x and w 16-byte aligned
 * and out 8-byte aligned; other shapes return hipErrorNotSupported and the caller quantizes +
 * GEMMs (the reference's order). K % 256 == 0. */
int cozyq_gemv(int device, const void* x, int x_half, const int8_t* w, const float* w_scale,
               const void* bias, void* out, int out_half, int M, int N, int K, void* stream);

/* A caller-provided scratch allocator (reference: gemm.cpp:55-67 `allocate`); may be NULL.
 * This build's GEMMs need no scratch and never call it. */
typedef void* (*cozyq_allocate_fn)(size_t bytes, void* context);

/* The quantized GEMM with the dequantizing epilogue (reference: gemm.cpp:127-145 `gemm`,
 * epilogue contract int8.h:65-71):
 *   out[m, n] = (acc[m, n] · scales[m]) · w_scale[n] (+ bias[n]),
 * acc the exact int32 (fp8 = 0, int8 q and w) or float32 (fp8 = 1, e4m3 q and w) sum over K.
 * int8: rounded as internal/int8_linear.py:445-448 + :276 (two float32 products, one cast,
 * then the bias added in the output dtype), bit-for-bit. fp8: float32 accumulation, one cast.
 * out rows are `ldo` elements apart (ldo >= N, ldo % 8 == 0, out 16-byte aligned); w_scale and
 * bias are 16-byte aligned. family must
 * be 0 (the one CDNA4 MFMA family). config names a tile as the reference's table does
 * (gemm_sm80.cu:233-289, gemm_fp8.cu:15-58), gfx950's own: 0 the 256x256 tile, 1 128x128,
 * 2 128x64, 3 64x64, 4 32x64, 5 256x192 (rows x columns); -1 chooses by shape
 * (cozyq_gemm_config; int8 at 1..4 rows with no epilogue activation takes a GEMV on the
 * quantized rows where K <= 32768 / 16384 / 12288 at 1 / 2 / 3..4 rows, and at 5..32 rows with
 * K <= 4096 and N <= 4096 a 16-row weight tile); 6 and above return
 * hipErrorNotSupported. Every config gives the same int8 output bit for bit.
 * N % 8 == 0; K % 256 (int8) or K % 16 (fp8). */
int cozyq_gemm(int device, int family, int fp8, const void* q, const float* scales,
               const void* w, const float* w_scale, const void* bias, void* out, int64_t ldo,
               int out_half, int M, int N, int K, int config, cozyq_allocate_fn allocate,
               void* allocate_context, void* stream);

/* The config cozyq_gemm (and cozyq_gemm_ex, which always chooses) runs for config -1 at this
 * shape (reference: the `choose` of gemm_sm80.cu:283-288 and gemm_fp8.cu:23-29, which the
 * reference does not export); -1 for a non-positive dimension. */
int cozyq_gemm_config(int fp8, int M, int N, int K);

/* cozyq_gemm with an epilogue activation (no reference counterpart: the reference's epilogue
 * is scales + bias only). epilogue 0: none; 1: tanh-GELU applied in float32 to the result of
 * cozyq_gemm's arithmetic, then cast. int8 K % 16 == 0 (any rotation lane). */
int cozyq_gemm_ex(int device, int fp8, const void* q, const float* scales, const void* w,
                  const float* w_scale, const void* bias, void* out, int64_t ldo, int out_half,
                  int M, int N, int K, int epilogue, void* stream);

/* The whole int8 linear in one launch: the reference's `quantize` then `gemm` (kernels/csrc/
 * gemm.cpp:83-117 and 119-168, chained by programmatic dependent launch, rotate.cu:284-295 and
 * gemm_tma.cuh:166-173) fused into one persistent kernel whose quantize jobs feed its GEMM tiles.
 * x [M, K] 16-bit (x_half: fp16, else bf16) is rotated (`rotation` 256: the reference's H256/16;
 * 128 and 0: the build's lanes of cozyq_quantize_rot) and quantized per row into q [M, K] int8 and
 * qs [M] f32 (the operand, which the caller may keep), then out = the int8 law of cozyq_gemm_ex
 * (epilogue 0 or 1) in x's dtype. K % max(rotation, 16) == 0, K <= 4096 (longer rows, or
 * out_half != x_half, return hipErrorNotSupported: run cozyq_quantize_rot + cozyq_gemm_ex).
 * N % 8 == 0, ldo >= N, ldo % 8 == 0; x, q, w and out 16-byte aligned. `workspace` holds
 * cozyq_linear_workspace_bytes(M) bytes, zero before the first call; each call leaves it zero, so
 * one workspace serves calls in stream order (calls that overlap on one workspace race). */
int64_t cozyq_linear_workspace_bytes(int64_t M);
int cozyq_linear(int device, const void* x, int x_half, int rotation, int8_t* q, float* qs,
                 const int8_t* w, const float* w_scale, const void* bias, void* out, int64_t ldo,
                 int out_half, int M, int N, int K, int epilogue, int* workspace, void* stream);

/* cozyq_linear that allocates nothing (no reference counterpart; for callers that cannot
 * allocate: code under graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments without `workspace`: the counters live in the library's own 4160-byte device array
 * (one per GPU, held until the process ends), cleared by a small kernel on `stream` ahead of each
 * launch. M <= cozyq_linear_noalloc_max_rows() (262144), else hipErrorInvalidValue before
 * anything runs. Every call on one GPU shares the array: calls that overlap on a GPU race. */
int cozyq_linear_noalloc_max_rows(void);

/* The fused linear's fault report (no reference counterpart: the reference's programmatic
 * dependent launch has no wait to give up). A tile waits for its rows' quantize jobs with a
 * bounded spin; a workgroup whose spin gives up writes NaN into every output tile it claims (never
 * a tile computed from codes that may not exist yet) and the launch records it in the counters'
 * status word. cozyq_linear_status synchronizes `stream`, returns hipErrorLaunchTimeOut if a call
 * on `workspace` gave up since the last read (and clears the record), else 0.
 * cozyq_linear_noalloc_status does the same for the allocation-free entry point's last call. */
int cozyq_linear_status(int device, int* workspace, void* stream);
int cozyq_linear_noalloc_status(int device, void* stream);
/* Test entry: the spin limit of later fused launches in this process (0 restores the default;
 * negative makes every wait give up at once, so the fault path runs with no wave waiting). */
void cozyq_linear_test_spin_limit(int limit);
int cozyq_linear_noalloc(int device, const void* x, int x_half, int rotation, int8_t* q, float* qs,
                         const int8_t* w, const float* w_scale, const void* bias, void* out,
                         int64_t ldo, int out_half, int M, int N, int K, int epilogue, void* stream);

/* Test entry (no reference counterpart): the raw int32 accumulators acc = q·wᵀ of the int8
 * GEMM, [M, N] row-major, for bit-exact checks of the MFMA mainloop. */
int cozyq_gemm_i32(int device, const int8_t* q, const int8_t* w, int32_t* acc, int M, int N,
                   int K, void* stream);

/* The w4a8.convrot GEMM (reference: gemm.cpp:147-157 `w4a8_gemm`, w4a8.cu): int8 q [M, K]
 * (int8.convrot's operand) times the int8 levels of 4-bit codes w [N, K/2] (even k in the low
 * nibble) with E4M3 group scales s [N, K/16] and a codebook of 16 float32 levels (NULL: the
 * uniform grid q - 8): level = clamp(rne(codebook[code] · e4m3(s)), ±127), a NaN product 0
 * (internal/prebuilt.py:471-492). The codes are unpacked in registers on the way to the int8
 * MFMA; the epilogue is cozyq_gemm's int8 law with w_scale [N], bit for bit. out [M, N].
 * N % 8 == 0, K % 256 == 0; q and w 16-byte aligned, out 8-byte aligned. config names
 * cozyq_gemm's narrow tiles 1..4 (-1: by rows, a GEMV form for 1..2 rows and a row-tile
 * kernel for 3..16 rows with K <= 8192 and 17..32 with K <= 4096 and M·K <= 98304, the same
 * bits); 0 and 5 (the 256-row tiles, which multiply
 * the codes unpacked by cozyq_w4a8_unpack) and 6 and above return hipErrorNotSupported. */
int cozyq_w4a8_gemm(int device, const int8_t* q, const float* scales, const uint8_t* w,
                    const uint8_t* s, const float* codebook, const float* w_scale, const void* bias,
                    void* out, int out_half, int M, int N, int K, int config, void* stream);

/* The same codes unpacked to their int8 levels, out [N, K] (reference: gemm.cpp:159-166
 * `w4a8_unpack`): the many-row path multiplies these on the int8 GEMM. w 8-byte aligned, out
 * 16-byte aligned. */
int cozyq_w4a8_unpack(int device, const uint8_t* w, const uint8_t* s, const float* codebook,
                      int8_t* out, int N, int K, void* stream);

/* The fp8 linear for few rows in one launch (no reference counterpart: the reference has no
 * fp8 GEMV, internal/fp8_linear.py:114-129 quantizes then multiplies): each row of x quantized
 * by cozyq_quantize's fp8 law inside the kernel, then out = acc·s_x·w_scale (+ bias).
 * M <= 4 with M·K <= 16384 (the GEMV), or 5 <= M <= 16 with K <= 4096 (the row-tile
 * kernel: one workgroup a CU, each owning 8-row units of N; 3 and 4 rows with M·N >= 36864 and
 * K <= 4096 take it too, faster there); K % 16 == 0; other shapes answer NOT_SUPPORTED (the
 * caller quantizes once and calls cozyq_gemm). */
int cozyq_fp8_linear(int device, const void* x, int x_half, const uint8_t* w,
                     const float* w_scale, const void* bias, void* out, int out_half, int M,
                     int N, int K, void* stream);

/* MXFP8 activation quantization (law: internal/encoding/leaves.py:1411-1424): per 32-block
 * of each row, byte = clamp(ceil(log2(amax/448)) + 127, 0, 254) (0 blocks: 0), elements
 * e4m3(clamp(x / 2^(byte-127), ±448)). q: [M, K] e4m3; scales: [M, K/32] E8M0, row-major.
 * K % 32 == 0. */
int cozyq_mx_quantize(int device, const void* x, int x_half, uint8_t* q, uint8_t* scales, int M,
                      int K, void* stream);

/* MXFP8 GEMM on the E8M0-scaled MFMA (reference: internal/encoding/leaves.py:1509-1519, which
 * calls cuBLASLt's `_scaled_mm` with 1x32 block scales):
 *   out[m, n] = Σ_k (q[m,k]·2^(qs[m,k/32]-127))·(w[n,k]·2^(ws[n,k/32]-127)) (+ bias[n]),
 * float32 accumulation, one cast. Scale grids are row-major [rows, K/32] (not cuBLAS's 128x4).
 * K % 128 == 0, N % 8 == 0, ldo as cozyq_gemm. */
int cozyq_mx_gemm(int device, const uint8_t* q, const uint8_t* q_scales, const uint8_t* w,
                  const uint8_t* w_scales, const void* bias, void* out, int64_t ldo, int out_half,
                  int M, int N, int K, void* stream);

/* SVDQuant W4A4 activation side, int4-g64 variant (reference: gemm.cpp:169-178
 * `svdq_quantize`, whose law is nvfp4): xs = bf16(x·p); per 64-group of each row
 * s = fp16(amax/7), code = clamp(rne(xs/s), -8, 7) (0 where s == 0), packed two a byte,
 * element 2k low: act [M, K/2], ascales [M, K/64] fp16. Also the low-rank input
 * la = bf16(x · downᵀ), down [R, K] bf16, la [M, R] bf16. K % 64 == 0, R in {16, 32, 64}. */
int cozyq_svdq_int4_quantize(int device, const void* x, int x_half, const float* p,
                             const void* down, uint8_t* act, uint16_t* ascales, void* la, int M,
                             int K, int R, void* stream);

/* SVDQuant W4A4 GEMM, int4-g64 variant (reference: gemm.cpp:180-190 `svdq_gemm`, svdq.cu:
 * 446-485): out = Σ_g (Σ_{k∈g} act·w)·ascales[m,g]·wscales[n,g] + la·upᵀ + bias, float32
 * accumulation, one cast. w [N, K/2] packed like act; wscales [N, K/64] fp16; up [N, R] bf16.
 * K % 64 == 0, N % 8 == 0; act, w, la, up and out 16-byte aligned, bias (if any) 4-byte. */
int cozyq_svdq_int4_gemm(int device, const uint8_t* act, const uint16_t* ascales,
                         const uint8_t* w, const uint16_t* wscales, const void* la,
                         const void* up, const void* bias, void* out, int out_half, int M, int N,
                         int K, int R, void* stream);

/* The rows svdq.nvfp4's activation operand is padded to, Rows(M) = M rounded up to 256
 * (reference: svdq.h:12-13 `kRows`, svdq_linear.py:48 NATIVE_ROWS); -1 for M < 0. */
int cozyq_svdq_rows(int M);

/* svdq.nvfp4's activation second level (reference: internal/svdq_linear.py:582-590
 * `activation_scale`, which takes it with torch ops): g[0] = max(max_{m,k} |x[m,k]|·p[k] / 2688,
 * 1e-30), float32, each product rounded, as the law's max over rows then columns. x [M, K]
 * 16-bit (x_half: fp16, else bf16), p [K] f32; both 16-byte aligned, K % 64 == 0. */
int cozyq_svdq_input_scale(int device, const void* x, int x_half, const float* p, int M, int K,
                           float* g, void* stream);

/* svdq.nvfp4 activation side (reference: gemm.cpp:169-178 `svdq_quantize`, svdq.h:27-33; law
 * internal/svdq_linear.py:592-618): xs = bf16(x·p); per 16-block of each row the E4M3 scale
 * e4m3(clamp(amax|xs| / (6·g[0]), 2^-9, 448)) and each element's E2M1 code (nearest, ties to the
 * even code, of |xs / (scale·g[0])|; sign in bit 3), two a byte with element 2k low. Layouts are
 * this build's (the reference's are its GEMM's fragment tiles; the sizes are the same):
 * act [Rows(M), K/2] and ascales [Rows(M), K/16] row-major, la = bf16(x·downᵀ) [Rows(M), R],
 * down [R, K] bf16 (cast to x's dtype for fp16 x); rows past M are zeros. K % 64 == 0,
 * R in {32, 64, 128}; every pointer 16-byte aligned. */
int cozyq_svdq_quantize(int device, const void* x, int x_half, const float* p, const float* g,
                        const void* down, void* act, void* ascales, void* la, int M, int K, int R,
                        void* stream);

/* svdq.nvfp4 GEMM (reference: gemm.cpp:180-190 `svdq_gemm`, svdq.h:35-42, svdq.cu:257-485):
 *   out[m, n] = (A·Wᵀ)[m, n]·gx[0]·gw[0]·c[n] + (la·upᵀ)[m, n] + bias[n], rounded once,
 * A from cozyq_svdq_quantize's act/ascales, W the stored nvfp4 weight: codes w [N, K/2] (element
 * 2k low) and E4M3 scales wscales [N, K/16], both row-major as stored (no retiling). Each element
 * is decoded exactly to fp16 and the products are summed in float32; the low-rank term enters the
 * same accumulators. up [N, R] bf16; c (f32 [N]) and bias (out's dtype) may be NULL. out [M, N]
 * bf16, or fp16 with out_half. M >= 1, N % 8 == 0, K % 64 == 0, R in {32, 64, 128}; every
 * pointer 16-byte aligned. */
int cozyq_svdq_gemm(int device, const void* act, const void* ascales, const void* w,
                    const void* wscales, const float* gx, const float* gw, const float* c,
                    const void* la, const void* up, const void* bias, void* out, int out_half,
                    int M, int N, int K, int R, void* stream);

/* Stored-format decode into a float destination (reference: the `decoded_float` providers of
 * internal/encoding/formats.py — TensorwiseDequant :438-488, RowwiseDequant :507-569,
 * MicroScaledDequant :588-650, Nvfp4Dequant :762-868 — and the nvfp4 decode core with its
 * per-column factor, internal/decode_schemes.py:362-431 and internal/decode_cores.py:196-230):
 *   out[e, i, j] = round(v · s · g)  (second 1),  round(v · (s / g))  (second 2),
 *   then · post (one factor or post[j]) before the rounding; each step a float32 rounding,
 *   one rounding (nearest even) into out.
 * v = value(w[e, i, j]) by `code`: 0 int8, 1 E4M3, 2 E5M2, 3 E2M1 packed two a byte (element 2k
 * in the low nibble, the high one with high_first). s = scale[grid(i, j)] by `grid`: 0 one
 * scale, 1 one per row, 2 one per column, 3 row blocks of `block` columns stored row-major
 * [rows, ceil(cols/block)] or, with `tiled`, in cuBLAS's 128x4 tiles (formats.py:154-178).
 * g = scale_2[e · scale_2_step]. Part dtypes (scale_type, post_type, out_type): 0 f32, 1 bf16,
 * 2 f16, 3 E8M0 (255 is NaN), 4 E4M3; out is f32, bf16 or f16. `matrices` stacked matrices of
 * [rows, cols] each, with a scale grid (row, block) and an optional scale_2 of their own. */
int cozyq_decode(int device, int code, const void* w, const void* scale, int scale_type, int grid,
                 int block, int tiled, const float* scale_2, int scale_2_step, int second,
                 const void* post, int post_type, int post_mode, int high_first, void* out,
                 int out_type, int64_t rows, int64_t cols, int matrices, void* stream);

/* int8.convrot decode (reference: Int8ConvRotDequant.decode, internal/encoding/formats.py:
 * 733-752): out[i, :] = round((H·w[i, g])·scale[i]·2^-k) for each rotation_size = 4^k group g,
 * H the regular H4⊗…⊗H4 (formats.py:657-671) summed exactly in int32. rotation_size in
 * 4 .. 65536, cols % rotation_size == 0; from 64 up, w and out 16-byte aligned. scale_type and
 * out_type as cozyq_decode (0-2). */
int cozyq_decode_convrot(int device, const int8_t* w, const void* scale, int scale_type,
                         int rotation_size, void* out, int out_type, int64_t rows, int64_t cols,
                         void* stream);

/* svdq.nvfp4 decode (reference: internal/decode_schemes.py:464-489): the nvfp4 value of
 * cozyq_decode (code 3, blocks of 16, E4M3 scales, second 1 or 2 by `divide`), · channel_scale[i]
 * (f32 or E4M3, optional), · smooth[j], then + up[i, r]·down[r, j] for r = 0 .. rank−1, each
 * product and sum rounded to float32, one rounding into out. w [rows, cols/2], scale
 * [rows, cols/16] (or tiled), smooth [cols], down [rank, cols], up [rows, rank]; cols % 16 == 0. */
int cozyq_decode_svdq(int device, const uint8_t* w, const uint8_t* scale, int tiled,
                      int high_first, const float* scale_2, int divide, const void* channel_scale,
                      int channel_type, const void* smooth, int smooth_type, const void* down,
                      int down_type, const void* up, int up_type, int rank, void* out,
                      int out_type, int64_t rows, int64_t cols, void* stream);

/* nvfp4 W4A16 GEMV for up to 64 rows (reference: the `_gemv` kernel of
 * internal/nvfp4_linear.py:126-201, which serves at most DECODE_ROWS = 16 rows, :338-377; past 16
 * rows the reference decodes and calls cuBLAS, :376-385, which this kernel replaces up to 64):
 *   out[m, n] = round((Σ_k x[m, k] · (e2m1[n, k] · scale[n, k/16])) · scale_2), float32 sums.
 * w [N, K/2] E2M1 codes, element 2k in the low nibble; scale E4M3 in cuBLAS's 128x4 tiles over
 * [N, K/16] (the leaf's resident layout); scale_2 one float32. x [M, K] bf16 or fp16 (x_half),
 * 16-byte aligned; out [M, N] bf16 or fp16. 0 ≤ M ≤ 64, K % 32 == 0. Past 4 rows, with K % 128 == 0
 * and at least 192 64-row groups in N, a row-block kernel runs (the activation read once per 64
 * weight rows); within each kernel a row's result does not
 * depend on M. */
int cozyq_nvfp4_gemv(int device, const void* x, int x_half, const uint8_t* w, const uint8_t* scale,
                     const float* scale_2, void* out, int out_half, int M, int N, int K, void* stream);

/* nvfp4 W4A16 GEMM for more rows (reference: the decode-then-cuBLAS path of
 * internal/nvfp4_linear.py:376-385 — `_dequant` into the activation dtype with scale_2 folded in,
 * then one library GEMM):
 *   out[m, n] = round((Σ_k x[m, k] · (e2m1[n, k] · scale[n, k/16])) · scale_2 + bias[n]),
 * float32 sums; the product e2m1 · E4M3 is exact in bf16 and fp16, so W is never rounded (the
 * reference rounds e2m1 · scale · scale_2 into x's dtype). The operands are nvfp4_gemv's, plus
 * bias [N] in out's dtype or null; x, w, scale, out and bias 16-byte aligned; M ≥ 0,
 * K % 64 == 0, N % 8 == 0. 256x256 output tiles. */
int cozyq_nvfp4_gemm(int device, const void* x, int x_half, const uint8_t* w, const uint8_t* scale,
                     const float* scale_2, const void* bias, void* out, int out_half, int M, int N, int K,
                     void* stream);

/* Weight encoders (reference: the tensorfs producers behind derive/microscale.py —
 * encode_int8_convrot256 :295-334, encode_fp8_rowwise :223-262, encode_w4a8 :349-408,
 * encode_nvfp4 :146-217 — whose arithmetic tensorfs holds; the laws here are this build's).
 * w is row-major [rows, K] of w_type 0 f32, 1 bf16, 2 f16, 16-byte aligned.
 * int8.convrot: r = H256(w)/16 (the reference's stage order), scale = max(amax/127, 1e-12),
 *   q = clamp(rne(r/scale), ±127); K % 256 == 0.
 * w4a8.convrot: int8.convrot's r and scale, t = r/scale; per 16-group group_scale =
 *   e4m3(max|t| / max|codebook|); each 4-bit code the nearest of clamp(rne(codebook[c]·σ), ±127)
 *   (first on a tie), even k in the low nibble: codes [rows, K/2], group_scale [rows, K/16].
 * fp8.rowwise: scale = max(amax/448, 1e-12), q = e4m3(clamp(w/scale, ±448)); K % 8 == 0.
 * mxfp8: per 32-block the MX law of cozyq_mx_quantize; E8M0 grid row-major [rows, K/32] or,
 *   with tiled, cuBLAS's 128x4 tiles (padding left as the caller filled it); K % 32 == 0.
 * nvfp4: scale_2 = amax(|w|)/2688 (1 for an all-zero matrix); per 16-block the E4M3 scale of
 *   e4m3(amax_b/(6·scale_2)) and its two neighbours with the least squared error, codes e2m1 of
 *   w/(scale·scale_2) to nearest even, saturated at ±6 and counted into `saturated`; low nibble
 *   first, row-major scales; `amax` and `saturated` zeroed by the caller; K % 16 == 0. */
int cozyq_encode_int8_convrot(int device, const void* w, int w_type, int8_t* q, float* scale,
                              int64_t rows, int K, void* stream);
int cozyq_encode_w4a8(int device, const void* w, int w_type, const float* codebook, uint8_t* codes,
                      uint8_t* group_scale, float* scale, int64_t rows, int K, void* stream);
int cozyq_encode_fp8_rowwise(int device, const void* w, int w_type, uint8_t* q, float* scale,
                             int64_t rows, int K, void* stream);
int cozyq_encode_mxfp8(int device, const void* w, int w_type, uint8_t* q, uint8_t* scale, int tiled,
                       int64_t rows, int K, void* stream);
int cozyq_encode_nvfp4(int device, const void* w, int w_type, uint8_t* codes, uint8_t* scale,
                       float* scale_2, uint32_t* amax, unsigned long long* saturated, int64_t rows,
                       int K, void* stream);

/* svdq.int4g64 weight producer (this build's W4A4 variant; the reference's svdq writer is
 * tensorfs's, not in the reference): v = float32((w − up·down) / p) with the residual and the
 * division in float64, then per 64-group s = fp16(amax|v| / 7) and codes clamp(rne(v / s), −8, 7)
 * (0 where s == 0), two a byte with element 2k low: codes [rows, K/2], scales [rows, K/64] fp16.
 * w [rows, K] f32 / bf16 / fp16 by w_type 0 / 1 / 2, p [K] f32, down [rank, K] and up [rows, rank]
 * bf16. K % 64 == 0; w, down, codes and scales 16-byte aligned. */
int cozyq_encode_svdq_int4(int device, const void* w, int w_type, const float* p, const void* down,
                           const void* up, int rank, uint8_t* codes, uint16_t* scales, int64_t rows,
                           int K, void* stream);

/* What an encoding lost (reference: the measured acceptance facts of derive/microscale.py:64-110,
 * `sse`, `energy`, `max_abs_err`): out = [Σ(w − d)², Σ w², max |w − d|] in float64 over `total`
 * elements of w (w_type as above) against its float32 decode d, folded through `parts`
 * float64 triples in `partial`. */
int cozyq_measure(int device, const void* w, int w_type, const float* decoded, int64_t total,
                  double* partial, int parts, double* out, void* stream);

/* LoRA bake, in place (reference: `fused`, internal/lora_bake.py:775-815, and its Triton kernel
 * `_bake_kernel`, :1013-1053, one entry for its five forms): data [rows, cols] takes
 * up [rows, rank] @ down [rank, cols] (float32, one FMA chain per element in rank order) and is
 * rounded back onto its form. form 0: bf16 (stochastic: 16 noise bits added under the kept
 * ones), 1: fp16, 2: float32 (nearest), 3: fp8.rowwise E4M3 bytes on the kept float32 row scale
 * `scale` [rows] (stochastic, saturating at 448), 4: int8.convrot (`down` already
 * `cozyq_bake_rotate_factor`ed; floor(code + delta/scale + u), clamped to ±127). Element (r, c)'s
 * noise is Philox4x32-10 at counter (r·cols + c mod 2^32, 0, 0, 0) under the key (seed, seed's
 * sign), Triton's `tl.randint` / `tl.rand`; the reference passes seed & 0x7FFFFFFF.
 * With gain, more and flags null / 0 this is the fused law exactly. The reference's eager bake
 * (`bake_plain` / `bake_rowwise` / `bake_int8_convrot`, :271-423) and `gain_rows` (:733-749) add:
 * `gain` float32 [rows] multiplying plain rows first (forms 0-2 only; a row-scaled weight takes
 * it in its scale), `more` float32 [rows, cols] added to the delta (a LoKr's dense rows; form 4:
 * rotated like `down`), flags 1 = round to nearest (ties to even) instead of stochastically,
 * 2 = no delta (the rows times their gain alone). `rescale` float32 [rows] (form 3 only) bakes
 * onto new row scales (`bake_rowwise`'s `refit` / `regrid` grids, :319-363): each code is the
 * rounding of (e4m3·scale + delta) / rescale, in the eager law's order; the caller stores
 * `rescale` as the new scale. data aligned to its element; rows ≤ 65535·64. Errors:
 * hipErrorInvalidValue for a bad form, shape, pointer, flag, a gain on forms 3-4 or a rescale
 * off form 3. */
int cozyq_bake(int device, int form, void* data, const float* scale, const float* up,
               const float* down, const float* gain, const float* more, const float* rescale,
               int64_t rows, int64_t cols, int64_t rank, uint32_t seed, int flags, void* stream);

/* LoRA bake into canonical nvfp4 (reference: `_bake_nvfp4_kernel`, internal/lora_bake.py:
 * 955-1011, `bake_nvfp4` with `keep`): codes [rows, cols/2] (element 2k in the low nibble), E4M3
 * block bytes [rows, cols/16] row-major, float32 second level at `second` (kept). A block keeps
 * its scale unless its baked maximum passes 7/6 of it, then takes the least E4M3 code that holds
 * it; elements round stochastically on the block's E2M1 grid (saturating at 6) with the noise of
 * `cozyq_bake`'s `tl.rand`; a zero keeps its stored sign. cols % 16 == 0. With gain, more or
 * flags (as `cozyq_bake`'s) the target follows the eager `bake_nvfp4` (:458-525): the decoded
 * value times the row's gain, plus the delta, each rounded. */
int cozyq_bake_nvfp4(int device, uint8_t* data, uint8_t* blocks, const float* second,
                     const float* up, const float* down, const float* gain, const float* more,
                     int64_t rows, int64_t cols, int64_t rank, uint32_t seed, int flags,
                     void* stream);

/* Each row's L2 norm of a stored weight plus up @ down (reference: `norms`, internal/lora_bake.py:
 * 653-689, DoRA's ||V||): out float32 [rows]. form as `cozyq_bake`'s, or 5 for nvfp4 (codes at
 * data, block bytes at `blocks`, level at `second`); form 4 takes `down` rotated. The sum of
 * squares is float64, in a fixed order. */
int cozyq_bake_norms(int device, int form, const void* data, const float* scale,
                     const uint8_t* blocks, const float* second, const float* up,
                     const float* down, int64_t rows, int64_t cols, int64_t rank, float* out,
                     void* stream);

/* Each row's max |decoded stored weight · gain + up @ down + more| (reference: the amax
 * `bake_rowwise`'s `refit` takes, internal/lora_bake.py:344-346, and `bake_nvfp4`'s, :495-500),
 * out float32 [rows]; `gain` float32 [rows] (plain and nvfp4 forms only) and `more` float32
 * [rows, cols] (LoKr's dense rows) or null; the other arguments as `cozyq_bake_norms`'s. A
 * maximum, so the same on every call. */
int cozyq_bake_row_amax(int device, int form, const void* data, const float* scale,
                        const uint8_t* blocks, const float* second, const float* up,
                        const float* down, const float* gain, const float* more, int64_t rows,
                        int64_t cols, int64_t rank, float* out, void* stream);

/* An nvfp4 bake with `grid="refit"` (reference: `bake_nvfp4`, internal/lora_bake.py:458-525):
 * the target decodes at the stored `second` level (e2m1·(e4m3(block)·second), plus delta); every
 * block's scale becomes the least E4M3 code at or above peak·(1/float(6·level)) and its elements
 * round on e4m3(block)·float(level). `level` is the new second level the caller takes from the
 * baked tensor's amax (amax / 2688 in double, 1 for all zeros) and then stores; flags 0
 * (stochastic, Philox counter row·cols + col) or 1 (nearest). data [rows, cols/2], blocks
 * [rows, cols/16] in place. `gain` float32 [rows] multiplies each decoded row and `more` float32
 * [rows, cols] adds to the delta (each may be null), as in `cozyq_bake_nvfp4`. */
int cozyq_bake_nvfp4_refit(int device, uint8_t* data, uint8_t* blocks, const float* second,
                           double level, const float* up, const float* down, const float* gain,
                           const float* more, int64_t rows, int64_t cols, int64_t rank, uint32_t seed,
                           int flags, void* stream);

/* An fp8.rowwise bake with error feedback (reference: `encode_e4m3(..., "feedback")`,
 * internal/lora_bake.py:163-197, under `bake_rowwise`): payload (e4m3·scale + delta) / fresh
 * (fresh = each row's scale after the bake: the kept one or a refitted one), each element
 * rounded to nearest E4M3 (saturating at 448) with the rounding error of the element before it
 * in its run of 32 columns added first; runs start at column multiples of 32. No noise. data
 * [rows, cols] E4M3 bytes in place; the caller stores `fresh` as the new scale. `more` float32
 * [rows, cols] (LoKr's dense rows) adds to the delta, or null. */
int cozyq_bake_feedback(int device, uint8_t* data, const float* scale, const float* fresh,
                        const float* up, const float* down, const float* more, int64_t rows,
                        int64_t cols, int64_t rank, void* stream);

/* A bake's accounting (reference: `Stats` and `_account`, internal/lora_bake.py:78-123,249-268):
 * the weight's parts before and after a bake (`before` / `after`, and for form 3-4 the row
 * scales, for form 5 the block bytes and `second`, the level `before` decodes at, and
 * `second_after`, the level `after` decodes at: null for `second`), with the gain, dense rows and factors the bake
 * took (form 4: `down` and `more` rotated). target = base + delta, decoded as the eager reference
 * decodes; partial receives 7 doubles per 64-row group, ceil(rows / 64) · 7 in all: Σ target²,
 * Σ delta², Σ (stored − target)², Σ (stored − base)·delta, the saturated count, Σ (delta @ downᵀ)²
 * and Σ ((stored − target) @ downᵀ)², each in a fixed order (any rank: the projections are taken
 * 128 ranks at a time). */
int cozyq_bake_stats(int device, int form, const void* before, const void* after,
                     const float* scale_before, const float* scale_after,
                     const uint8_t* blocks_before, const uint8_t* blocks_after, const float* second,
                     const float* second_after, const float* gain, const float* more, const float* up,
                     const float* down, int64_t rows, int64_t cols, int64_t rank, double* partial,
                     void* stream);

/* `down` [rank, cols] in an int8-convrot256/1 weight's basis (reference: `rotate_factor`,
 * internal/lora_bake.py:366-369): each 256 columns times the regular Hadamard H4⊗H4⊗H4⊗H4 in
 * the expression order of internal/encoding/formats.py:664-671, then 1/16; out [rank, cols]
 * float32. cols % 256 == 0. */
int cozyq_bake_rotate_factor(int device, const float* down, float* out, int64_t rank,
                             int64_t cols, void* stream);

/* Test entries (no reference counterpart): the kernels' scalar conversions run on the host,
 * so CPU tests can hold the device code's arithmetic against torch without a GPU. */
void cozyq_host_e4m3(const float* in, uint8_t* out, int64_t n);
void cozyq_host_mx_byte(const float* amax, uint8_t* out, int64_t n);

/* Test entry (no reference counterpart): float32 -> E4M3 bytes through gfx950's hardware
 * conversion (v_cvt_pk_fp8_f32), n even, to hold it against the software encoder. */
int cozyq_probe_e4m3(int device, const float* in, uint8_t* out, int64_t n, void* stream);

/* Test entry (no reference counterpart): float32 values, taken as quotients xs / (scale·g), ->
 * the svdq.nvfp4 quantizer's E2M1 codes (v_cvt_scalef32_pk_fp4_f32 after its −0 and NaN
 * fix-ups), two a byte, the first in the low nibble; n even. Holds the conversion against the
 * law's threshold count (internal/svdq_linear.py:612-616). */
int cozyq_probe_e2m1(int device, const float* in, uint8_t* out, int64_t n, void* stream);

/* Test entry (no reference counterpart): x / s through the quantizers' reciprocal-and-correction
 * division, to hold it against IEEE division. */
int cozyq_probe_div(int device, const float* x, const float* s, float* out, int64_t n,
                    void* stream);

/* Test entry (no reference counterpart): one MFMA on per-lane operands, to confirm the lane
 * layouts the GEMMs rely on. kind 0: i32_16x16x64_i8 (a, b: 64 lanes x 16 bytes);
 * 1: f32_16x16x128_f8f6f4 e4m3 (64 lanes x 32 bytes); 2: the same with E8M0 scales sa, sb
 * (one byte a lane); 3: f32_16x16x32_bf16 (64 lanes x 16 bytes); 4: i32_32x32x32_i8 (64 lanes
 * x 16 bytes); 5: f32_32x32x64_f8f6f4 e4m3 (64 lanes x 32 bytes); 6: the same with E8M0
 * scales; 7: f32_32x32x2_f32 (one float a lane, the first 4 bytes); 8: f32_32x32x16_f16 (64
 * lanes x 16 bytes). a and b are read as 64 lanes x 32 bytes; d receives 64 lanes x 16
 * int32/float32 words (the 16x16 kinds fill the first 4). */
int cozyq_probe_mfma(int device, int kind, const void* a, const void* b, const void* sa,
                     const void* sb, void* d, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* COZYQ_H */
