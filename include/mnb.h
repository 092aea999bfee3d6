/*
 * mnb.h -- C ABI of the MI355X MatMulNBits (com.microsoft, bits = 4) library.
 *
 * The library implements the operator the onnx-light-cpu roadmap plans as
 * `int4_gemv` / `int4_small_m` / `int4_gemm` behind a prepared weight-only plan
 * (docs/next_steps/2026/2026_08_qwen3_inference.rst:188-230, 400-419, 530-540).
 * The reference has no GPU and no C ABI; each entry point below names the
 * reference interface whose role it takes over.
 *
 * Conventions
 *  - Plain C types only. Streams are passed as `void*` holding a hipStream_t
 *    (NULL = the default stream).
 *  - Every entry point returns an mnb_status; nothing throws across the ABI.
 *    Argument validation happens before any HIP call, so bad shapes and null
 *    pointers are reported without touching the GPU.
 *  - A plan is immutable after creation. mnb_run is reentrant for distinct
 *    output and workspace buffers; the plan's device constants are shared.
 *
 * Operator contract (ONNX Runtime contrib op, the layout this library keeps):
 *   A      fp32 [M, K] row-major (device memory)
 *   B      uint8 [N, nb, block_size/2], nb = ceil(K / block_size); element
 *          k = b*block_size + j of row n is nibble j of B[n, b, :], low nibble
 *          first (onnx_light_cpu/impl/math/gemm/vnni/integer_gemm_vnni.h:42-51)
 *   scales fp32 [N, nb]
 *   zero_points uint8 [N, ceil(nb/2)], nibble b of row n, low nibble first;
 *          absent means 8
 *   Y      fp32 [M, N] = A * W^T, W[n,k] = (q - zp) * scale
 */
#ifndef MNB_H
#define MNB_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mnb_status {
  MNB_OK = 0,
  MNB_ERR_NULL_POINTER = 1,     /* a required pointer is NULL */
  MNB_ERR_BAD_SHAPE = 2,        /* K, N or M out of range */
  MNB_ERR_BAD_ATTRIBUTE = 3,    /* block_size not a power of two >= 16, bad accuracy_level */
  MNB_ERR_UNSUPPORTED = 4,      /* bits != 4, or an input this version rejects */
  MNB_ERR_WORKSPACE = 5,        /* workspace smaller than mnb_workspace_bytes */
  MNB_ERR_HIP = 6,              /* a HIP runtime call failed */
  MNB_ERR_NO_DEVICE = 7,        /* no gfx950 device is current */
  MNB_ERR_ALLOC = 8             /* device allocation failed */
} mnb_status;

/* Node attributes and optional-input presence of one MatMulNBits node.
 * Replaces what KernelBase reads from the NodeProto in the reference's
 * operator wrappers (onnx_light_cpu/kernels/math/gemm_kernel.cc:470-473 for
 * attributes, integer_matmul_kernel.cc:375-376 for optional inputs). */
typedef struct mnb_desc {
  int64_t K;                /* attribute K */
  int64_t N;                /* attribute N */
  int32_t bits;             /* attribute bits: 4 only */
  int32_t block_size;       /* attribute block_size: power of two >= 16 */
  int32_t accuracy_level;   /* attribute accuracy_level, 0..4: 1 keeps fp32 activations on
                               every path (see mnb_run) */
  int32_t has_zero_points;  /* input 3 present */
} mnb_desc;

typedef struct mnb_plan mnb_plan;

/* Prepared plan: validates the attributes and uploads the constant B, scales
 * and zero points (host pointers) to the current device once; the plan owns
 * the device copies. Replaces the reference's prepared plan with a constant B
 * (MatMulPlan constant_b, onnx_light_cpu/impl/math/gemm/gemm_plan.h:161-195;
 * GemmPlanOptions::constant_b, gemm_plan.h:34-38). zero_points must be NULL
 * when desc->has_zero_points == 0. Plan creation allocates device memory and
 * waits for its own copies and re-layout kernels: create plans before, not
 * during, the capture of a stream of the device into a HIP graph. */
int mnb_plan_create(const mnb_desc *desc, const uint8_t *B, const float *scales,
                    const uint8_t *zero_points, mnb_plan **out_plan);

/* Same as mnb_plan_create, but B, scales and zero_points are device pointers
 * on the current device that the plan borrows: the caller keeps them alive
 * and unchanged for the plan's lifetime. The call first waits for all work
 * already issued on the device (hipDeviceSynchronize), so writes to the
 * buffers on any stream must have been issued before it; it then derives the
 * plan's own re-laid copies from the buffers' contents at that point (the
 * kernels read those copies, so later changes to the buffers are not seen
 * by every path). */
int mnb_plan_create_device(const mnb_desc *desc, const uint8_t *dB, const float *dScales,
                           const uint8_t *dZeroPoints, mnb_plan **out_plan);

/* Gated-MLP front half as one plan: H[M, N] = silu(A * Wg^T) (*) (A * Wu^T),
 * silu(x) = x * sigmoid(x), for a gate weight (Bg, Sg, Zg) and an up weight
 * (Bu, Su, Zu) that share desc (K, N = intermediate size, block_size,
 * zero-point presence; host pointers, MatMulNBits layout each). The graph
 * fusion the roadmap lists as "gate projection, SiLU, and gate/up
 * multiplication" over two MatMulNBits nodes, a Sigmoid and two Muls
 * (docs/next_steps/2026/2026_08_qwen3_inference.rst:371-377); the unfused
 * graph stays the correctness reference. The plan re-lays the rows once, at
 * creation (row 2n = gate row n, row 2n + 1 = up row n), so each pair meets
 * in one wavefront. mnb_run / mnb_run_path / mnb_run_ex on it write H
 * (M x N floats); bias is rejected (MNB_ERR_UNSUPPORTED). The workspace
 * (mnb_workspace_bytes) starts with the M x 2N fp32 sum that the kernels
 * whose epilogue cannot apply the activation write (followed by a separate
 * pass); it is required on every path except the decode path where the
 * fragment-ordered M <= 4 GEMV serves the plan (its epilogue applies the
 * activation). */
int mnb_plan_create_gate_up(const mnb_desc *desc, const uint8_t *Bg, const float *Sg,
                            const uint8_t *Zg, const uint8_t *Bu, const float *Su,
                            const uint8_t *Zu, mnb_plan **out_plan);

/* Releases the plan and the device memory it owns. NULL is accepted. */
int mnb_plan_destroy(mnb_plan *plan);

/* Device bytes the plan owns: its copy of the constants where it keeps one
 * (not borrowed buffers), the per-row scale exponents and the re-laid copies.
 * A plan created from host weights whose every path runs on the re-laid
 * copies (wide weights: N / 64 row groups covering most CUs, K % 256 == 0,
 * K <= 8192, 32 <= block_size <= 256) keeps no original layout ("compact":
 * about 1.07x the constants' bytes at block_size 128 with zero points);
 * others keep both (about 2.07x). No counterpart in the reference (whose
 * constant B stays in host memory): for callers planning device memory. */
int mnb_plan_device_bytes(const mnb_plan *plan, size_t *bytes);

/* Device workspace (16-byte aligned) that mnb_run and mnb_run_path need for M
 * rows, whichever path serves them (0 when none): the larger of
 *  - the prefill GEMM's: A scaled per row by a power of two and rounded to
 *    fp16 in its tile layout, ceil(M/128)*128*K*2 bytes, the rows' exponents
 *    (ceil(M/128)*128 int32, rounded up to 256 bytes), then, when the GEMM
 *    splits K into S > 1 parts, (S - 1)*M*N*4 bytes of fp32 partial sums
 *    (S <= 16, chosen from the shape);
 *  - where an MFMA decode kernel with a workspace serves min(M, 16) rows
 *    (5 <= M <= 16, from M = 4, 3 or 2 for wide weights, as mnb_run; the
 *    exact route serves larger M 16 rows at a time), its split activation
 *    image and fp32 partial sums (none where the fragment-ordered M <= 4
 *    GEMV serves them);
 *  - for 1 or 2 rows too long for one workgroup per 64-row group (K > 16384
 *    at M = 1, K > 8192 at M = 2; plain plans), the fragment-ordered GEMV
 *    with K split into S segments: (S - 1)*M*N*4 bytes of partial sums;
 *  - on a gate/up plan, plus the M x 2N fp32 scratch sum.
 * Without it (NULL or smaller) the decode path runs its fp32-FMA kernels. */
int mnb_workspace_bytes(const mnb_plan *plan, int64_t M, size_t *bytes);

/* Y = MatMulNBits(A, plan) for M rows; dA and dY are device pointers on the
 * plan's device. M == 0 is a no-op. Replaces the operator's compute call,
 * MatMulKernel::operator() -> MatMulPlan<float>::Execute
 * (onnx_light_cpu/kernels/math/matmul_kernel.cc:117-134, gemm_plan.cc:539-570).
 * M <= 4 on plans whose 64-row groups cover most CUs: decode GEMV on fp16
 * MFMA (A split into three fp16 terms after a power-of-two scaling per 256-k
 * unit, nibbles as fp16 subnormals; fp32 sums within about 2^-22 of
 * sum |a w| per output); other M = 1 plans: fp32 mixed-FMA GEMV; M <= 4 otherwise: fp32-FMA
 * decode GEMV; 5 <= M <= 16 (from M = 4 when N >= 3K, M = 3 when N >= 6K):
 * decode GEMV on fp16 MFMA with A split into two fp16 terms (22 bits) after
 * a power-of-two scaling, exact q - zp, fp32 sums;
 * M > 16: fp16-MFMA prefill GEMM. Its A row m is scaled by a power of two
 * 2^f_m (largest magnitude in [2^14, 2^15)) and rounded to fp16 (round to
 * nearest even, half_conversion.h:42-78); each weight row's block scales are
 * scaled by a power of two at plan time so they are normal fp16 numbers; the
 * fp32 epilogue undoes both exactly. No finite input overflows.
 * accuracy_level (ONNX Runtime's minimum accuracy of A: 0 unset, 1 fp32,
 * 2 fp16, 3 bf16, 4 int8): at level 1, M > 16 runs the exact-product decode
 * kernels 16 rows at a time (path 4) instead of the fp16 GEMM; levels 0
 * (unset, this library's default) and 2-4 take the GEMM, whose 11-bit
 * activations meet what levels 2-4 permit. M > 16 with K an odd multiple
 * of 32, which the GEMM kernels do not take, runs path 4 at every level;
 * K not a multiple of 32 runs the generic kernel (path 3). The launch is
 * asynchronous on `stream`. */
int mnb_run(const mnb_plan *plan, int64_t M, const float *dA, float *dY, void *dWorkspace,
            size_t workspace_bytes, void *stream);

/* Same as mnb_run with the kernel chosen by the caller (whatever the plan's
 * accuracy_level): path 0 = automatic, 1 = decode GEMV (any M <= 16),
 * 2 = MFMA GEMM (any M; the kernel picked by shape), 3 = generic fallback
 * (any shape; slow, for cross-checks), 4 = the decode kernels over
 * consecutive groups of 16 rows (any M; the exact route of accuracy_level 1),
 * 5 = the MFMA GEMM's prefill kernel over the plan's fragment-ordered weight
 * copy (any M; MNB_ERR_UNSUPPORTED when the plan holds none: K % 64 != 0,
 * N % 4 != 0, block_size < 32 or N >= 2^22). */
int mnb_run_path(const mnb_plan *plan, int64_t M, const float *dA, float *dY, void *dWorkspace,
                 size_t workspace_bytes, void *stream, int path);

/* Same as mnb_run_path, plus MatMulNBits' optional input 5: dBias, fp32 [N]
 * in device memory (NULL = absent), added to every row of Y:
 * Y = A * W^T + bias. Replaces the bias input the reference's operator
 * wrappers read as an optional input (integer_matmul_kernel.cc:375-376,
 * GetInput returning null when absent). */
int mnb_run_ex(const mnb_plan *plan, int64_t M, const float *dA, const float *dBias, float *dY,
               void *dWorkspace, size_t workspace_bytes, void *stream, int path);

/* RMSNorm into the projection input: Y = MatMulNBits(RMSNormalization(X)),
 * RMSNormalization(X)[m][k] = X[m][k] / sqrt(mean_k(X[m][k]^2) + epsilon)
 * * gamma[k] (ONNX RMSNormalization-23 over the last axis with fp32 stash,
 * the schema the roadmap targets: docs/next_steps/2026/2026_08_qwen3_inference.rst:143, 282),
 * fused as the roadmap's "RMSNorm into packed projection input" (:371-373).
 * dX fp32 [M, K] and dGamma fp32 [K] are device pointers, 16-byte aligned,
 * K % 4 == 0 (else MNB_ERR_UNSUPPORTED); epsilon >= 0. Decode path: the
 * M = 1 GEMV and the M <= 4 fragment-ordered GEMV in one kernel (each
 * reduces its rows' mean squares while staging them); the small-M MFMA
 * decode in its own two launches (the activation split multiplies by gamma
 * and sums x^2 per 256-k unit, the main kernel scales each row's sums by
 * 1/rms); the GEMM path: a per-row 1/rms pass, then gamma and 1/rms folded
 * into the GEMM's conversion of A to fp16; every other kernel (the fp32-FMA
 * decode fallbacks): the normalized input is written to the workspace first. Works on gate/up plans too (H of the
 * normalized input). The workspace is required:
 * mnb_rmsnorm_workspace_bytes. */
int mnb_rmsnorm_workspace_bytes(const mnb_plan *plan, int64_t M, size_t *bytes);
int mnb_run_rmsnorm(const mnb_plan *plan, int64_t M, const float *dX, const float *dGamma,
                    float epsilon, float *dY, void *dWorkspace, size_t workspace_bytes,
                    void *stream);

/* Bytes of the device scratch array behind mnb_run_no_alloc (32 MiB). */
#define MNB_NO_ALLOC_SCRATCH_BYTES (32u << 20)

/* mnb_run without a caller workspace and without any allocation: the
 * kernels' workspace is a fixed device array of MNB_NO_ALLOC_SCRATCH_BYTES
 * inside the library, one copy per GPU, held until the process ends (its
 * address is looked up on the first call on each device). No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Fails with MNB_ERR_WORKSPACE, before any launch, when the
 * workspace of the kernels mnb_run would launch for these M rows (at most
 * mnb_workspace_bytes(plan, M); e.g. the prefill GEMM above M * K * 2 of
 * about 32 MiB, or a gate/up plan's M x 2N scratch sum) exceeds the array. Every
 * call on a GPU shares that GPU's array: calls that overlap in time on one
 * GPU (several streams or threads) race and must be ordered by the caller.
 * No kernel reads scratch bytes it did not write in the same call, so the
 * previous call's leftovers never reach a result. */
int mnb_run_no_alloc(const mnb_plan *plan, int64_t M, const float *dA, float *dY, void *stream);

/* Which path mnb_run takes for M rows (1 to 4 as in mnb_run_path; the
 * automatic GEMM path reports 2 whichever GEMM kernel serves). */
int mnb_select_path(const mnb_plan *plan, int64_t M, int *path);

/* Kernels a run can launch, for mnb_kernel_name and mnb_run_kernel. */
#define MNB_KERNEL_GEMV_M1 1      /* GemvM1Kernel: M = 1, fp32 mixed FMA */
#define MNB_KERNEL_GEMV_SMALL_M 2 /* GemvSmallMKernel: 2 <= M <= 16, fp32 FMA */
#define MNB_KERNEL_GEMV_MFMA 3    /* GemvMfmaKernel: 2 <= M <= 16, exact-product MFMA, original layout */
#define MNB_KERNEL_DECODE_FRAG 4  /* DecodeFragKernel: 2 <= M <= 16, exact-product MFMA, fragment-ordered copy */
#define MNB_KERNEL_GEMM 5         /* GemmKernel: fp16 MFMA, BM x 128 tiles, original layout */
#define MNB_KERNEL_PREFILL 6      /* PrefillKernel: fp16 MFMA, 128 x 256 tiles, fragment-ordered copy */
#define MNB_KERNEL_GEMV 7         /* GemvKernel: fp32 FMA fallback, M <= 16 */
#define MNB_KERNEL_GENERIC 8      /* GenericKernel: any shape, one wavefront per output */
#define MNB_KERNEL_STREAM 9       /* StreamKernel: 17 <= M <= 64, fp16 MFMA, fragment-ordered copy streamed once */
#define MNB_KERNEL_GEMV_FRAG 10  /* GemvFragKernel: M <= 4, fp16 MFMA on nibble subnormals, fragment-ordered copy, A staged in LDS */

/* Name of the main kernel mnb_run launches for M rows given workspace_bytes
 * of workspace ("GemvM1Kernel", "DecodeFragKernel", "PrefillKernel", ...;
 * "" for M == 0 or a bad plan). Static storage. The counterpart of the
 * reference's record of the kernels a run dispatched to
 * (onnx_light_cpu/_register.py:157-170, used_kernel_names), answered before
 * the run. */
const char *mnb_kernel_name(const mnb_plan *plan, int64_t M, size_t workspace_bytes);

/* Tuning and cross-checks: one run of M rows with the named kernel (one of
 * MNB_KERNEL_*) and launch shape p0, p1 (0 picks each): GEMV_M1 (band rows,
 * rows per wavefront), GEMV_SMALL_M (tokens per launch, wavefronts per
 * workgroup), GEMV_MFMA (16-row blocks per item, workgroups per CU),
 * DECODE_FRAG (wavefronts per workgroup, 256-k units per wavefront), GEMM
 * (tile height 32, 64 or 128; K splits), PREFILL (K splits), STREAM (K
 * segments, 32-k steps per wavefront; both or neither), GEMV_FRAG
 * (32-k steps per wavefront: 8, 16 or 32; weight records in flight per
 * wavefront: 4 or 8; for M > 1 only 8 or 16 steps and 8 records); GEMV and
 * GENERIC take none. Plain (not gate/up) plans, no bias; MNB_ERR_UNSUPPORTED
 * when the kernel cannot serve the plan or M, MNB_ERR_WORKSPACE below
 * mnb_kernel_workspace_bytes. No counterpart in the reference, whose
 * kernels are chosen inside the plan. */
int mnb_kernel_workspace_bytes(const mnb_plan *plan, int64_t M, int kernel, int p0, int p1,
                               size_t *bytes);
int mnb_run_kernel(const mnb_plan *plan, int64_t M, const float *dA, float *dY, void *dWorkspace,
                   size_t workspace_bytes, void *stream, int kernel, int p0, int p1);

/* Words of dOut that mnb_stream_read writes (one per wavefront). */
#define MNB_STREAM_OUT_WORDS 2048u

/* HBM read ceiling probe: one launch that streams `bytes` (< 2^31) of device
 * memory at dSrc and nothing else (2048 wavefronts, each reading 8 KiB
 * contiguous records with eight 16-byte loads in flight), folding them into
 * dOut[0 .. MNB_STREAM_OUT_WORDS) so the loads are kept. A decode launch's
 * roofline fraction is reported next to this probe's rate over the same
 * bytes per launch. No counterpart in the reference. */
int mnb_stream_read(const void *dSrc, size_t bytes, uint32_t *dOut, size_t out_words,
                    void *stream);

/* The same probe on a given grid: `workgroups` workgroups of `threads`
 * threads (a multiple of 64, at most 1024), each wavefront reading one
 * contiguous share of the bytes (rounded up to 1 KiB) with eight 16-byte
 * loads in flight, one word per wavefront into dOut (out_words >= the
 * wavefront count, at most 65536). It gives the read rate a decode kernel's
 * own grid allows, e.g. one workgroup of 8 wavefronts per 64-row group. No
 * counterpart in the reference. */
int mnb_stream_read_grid(const void *dSrc, size_t bytes, uint32_t *dOut, size_t out_words,
                         int workgroups, int threads, void *stream);

/* Text for a status code (static storage). */
const char *mnb_status_str(int status);

/* Text of the last HIP error seen by this thread ("" if none). */
const char *mnb_last_error(void);

/* Bytes a plan with this description reads per call beyond A and Y
 * (packed B + fp32 scales + packed zero points): the algorithmic weight
 * bytes of one launch. */
int mnb_weight_bytes(const mnb_desc *desc, size_t *bytes);

/* QDQ front-end: repacks a constant weight-only DequantizeLinear feeding
 * MatMul(A, W) -- W[K, N] = DequantizeLinear(x, x_scale, x_zero_point) with
 * blocked quantization along axis 0 (K), the roadmap's qwen3-int4-qdq export
 * contract (docs/next_steps/2026/2026_08_qwen3_inference.rst:96-101, 262) --
 * into MatMulNBits inputs on the host, without forming any float weight:
 *   x            INT4 (is_signed = 1) or UINT4 [K, N], ONNX packing: element
 *                i of the row-major flattening is nibble i & 1 of byte i / 2,
 *                low nibble first, signed nibbles two's complement
 *                (onnx_light_cpu/impl/math/gemm/vnni/integer_gemm_vnni.h:42-47,
 *                ReadPacked4Bit integer_gemm_vnni.cc:60-65)
 *   x_scale      fp32 [ceil(K / block_size), N]
 *   x_zero_point same type and packing as x, [ceil(K / block_size), N], or
 *                NULL (ONNX default 0)
 * Outputs (caller-allocated, host memory): B [N, nb, block_size/2] (padding
 * nibbles past K are 0), scales [N, nb], zero_points [N, ceil(nb/2)], and
 * *has_zero_points: 0 when every zero point is the MatMulNBits default 8
 * (INT4 without x_zero_point; zero_points is then left untouched), else 1.
 * A signed nibble x maps to x + 8 and its zero point z to z + 8, so
 * (x - z) is unchanged. block_size must be a power of two >= 16. */
int mnb_qdq_repack(int64_t K, int64_t N, int32_t block_size, int32_t is_signed,
                   const uint8_t *x, const float *x_scale, const uint8_t *x_zero_point,
                   uint8_t *B, float *scales, uint8_t *zero_points, int32_t *has_zero_points);

/* Library version string. */
const char *mnb_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MNB_H */
