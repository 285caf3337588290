/*
 * fp8_blockwise.h -- C ABI of the MI355X (gfx950) block-FP8 linear path.
 *
 * Two stages, each a hand-written HIP kernel family in libfp8_blockwise.so:
 *   1. per-token-group activation quantisation: bf16 (or fp16, fp32) [M,K] ->
 *      float8_e4m3fn [M,K] plus fp32 scales [M, ceil(K/group)], scale = amax/448;
 *   2. w8a8 GEMM  C[M,N] = A[M,K] . B[N,K]^T  with A carrying per-(row, K-block)
 *      fp32 scales As and B carrying per-(N-block, K-block) fp32 scales Bs,
 *      accumulated in fp32 and stored as fp32, bf16 or fp16.
 *
 * Conventions shared by every entry point:
 *   - all data pointers are DEVICE pointers; the library never allocates,
 *     frees or copies on the host; it only reads/writes the caller's buffers;
 *   - strides are in ELEMENTS, the innermost (K or N) stride of matrices is 1;
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream);
 *     launches are asynchronous on it; the functions are stateless and
 *     re-entrant (concurrent calls on different streams are safe);
 *   - the return value is an fp8b_status; no C++ exception crosses the ABI.
 *     fp8b_last_error() returns a static text describing the last failure of
 *     the calling thread.
 */
#ifndef FP8_BLOCKWISE_H
#define FP8_BLOCKWISE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum fp8b_status {
  FP8B_OK = 0,
  FP8B_ERR_NULL = 1,       /* a required pointer is NULL                         */
  FP8B_ERR_DIMS = 2,       /* negative/overflowing size or stride                */
  FP8B_ERR_ALIGN = 3,      /* pointer or leading dimension misaligned             */
  FP8B_ERR_BLOCK = 4,      /* unsupported block_n / block_k / group size          */
  FP8B_ERR_DTYPE = 5,      /* unsupported output dtype code                       */
  FP8B_ERR_WORKSPACE = 6,  /* workspace too small for the chosen plan             */
  FP8B_ERR_LAUNCH = 7      /* a HIP launch or runtime call failed                 */
} fp8b_status;

/* Output element type codes for the GEMM epilogue. */
typedef enum fp8b_dtype {
  FP8B_F32 = 0,
  FP8B_BF16 = 1,
  FP8B_F16 = 2
} fp8b_dtype;

/* Library version, e.g. 0x000100 = 0.1.0. */
int fp8b_version(void);

/* Text of the calling thread's most recent error (never NULL). */
const char* fp8b_last_error(void);

/*
 * Per-token-group fp8 quantisation.
 *
 * No counterpart exists in the reference: finegrained-fp8-helion consumes
 * already-quantised A/As (torch-ext/finegrained_fp8_helion/fp8.py:5,24) and
 * ships no quantiser. The contract is the one its callers feed it with:
 *   for each row m and group g = [g*group, min((g+1)*group, K)):
 *     amax   = max |x[m,k]|          (NaN if any element is NaN)
 *     amax'  = max(amax, 1e-10)
 *     s[m,g] = amax' / 448            (fp32, IEEE division)
 *     q[m,k] = float8_e4m3fn(x[m,k] / s[m,g])   (IEEE division, RNE)
 *   non-finite groups: amax NaN -> s = NaN, every q = 0x7F;
 *                      amax +inf -> s = +inf, q = signed zero for finite x,
 *                      0x7F for +-inf.
 *
 * x : bf16 [M,K] with row stride ldx; q : e4m3fn [M,K] row stride ldq;
 * s : fp32, element (m,g) at s[m*s_stride_m + g*s_stride_g].
 * group must be 32, 64, 128 or 256.
 */
int fp8b_act_quant(const void* x, int64_t ldx,
                   void* q, int64_t ldq,
                   float* s, int64_t s_stride_m, int64_t s_stride_g,
                   int64_t M, int64_t K, int64_t group,
                   void* stream);

/*
 * fp8b_act_quant for x of x_dtype FP8B_F32, FP8B_BF16 or FP8B_F16 (ldx in
 * elements of x_dtype), with the same contract on the fp32 values of x (every
 * fp16 and bf16 value is exact in fp32). FP8B_BF16 is fp8b_act_quant. No
 * counterpart in the reference (see fp8b_act_quant); it serves callers whose
 * activations are not bf16.
 */
int fp8b_act_quant_typed(const void* x, int64_t ldx, int x_dtype,
                         void* q, int64_t ldq,
                         float* s, int64_t s_stride_m, int64_t s_stride_g,
                         int64_t M, int64_t K, int64_t group,
                         void* stream);

/*
 * Block-scaled w8a8 GEMM: C = A . B^T.
 *
 * Replaces the Helion kernel _w8a8_block_fp8_matmul
 * (finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/fp8.py:19-39)
 * behind the custom op of op.py:8-11:
 *   C[m,n] = sum_kb ( sum_{k in kb} A[m,k] B[n,k] ) * As[m,kb] * Bs[n/block_n, kb]
 *
 * A  : e4m3fn [M,K], row stride lda      B  : e4m3fn [N,K], row stride ldb
 * As : fp32, (m,kb) at As[m*as_sm + kb*as_sk]
 * Bs : fp32, (nb,kb) at Bs[nb*bs_sn + kb*bs_sk]
 * C  : out_dtype [M,N], row stride ldc
 * kb runs over ceil(K/block_k) K-blocks; nb over ceil(N/block_n).
 *
 * block_n = block_k = 128, K % 128 == 0, 16-byte aligned A/B with lda, ldb
 * multiples of 16 take the MFMA path; any other positive block sizes take a
 * generic (slower) GPU kernel with the same semantics.
 * workspace may be NULL when fp8b_gemm_workspace_size() returns 0 for the
 * same arguments; otherwise it must hold at least that many bytes.
 */
int fp8b_w8a8_block_matmul(const void* A, int64_t lda,
                           const void* B, int64_t ldb,
                           const float* As, int64_t as_sm, int64_t as_sk,
                           const float* Bs, int64_t bs_sn, int64_t bs_sk,
                           void* C, int64_t ldc, int out_dtype,
                           int64_t M, int64_t N, int64_t K,
                           int64_t block_n, int64_t block_k,
                           void* workspace, size_t workspace_bytes,
                           void* stream);

/* Bytes of device workspace fp8b_w8a8_block_matmul needs for these sizes. */
size_t fp8b_gemm_workspace_size(int64_t M, int64_t N, int64_t K,
                                int64_t block_n, int64_t block_k);

/* Kernels of the GEMM plans (fp8b_plan_info.kernel, .tail_kernel). */
typedef enum fp8b_kernel {
  FP8B_KERNEL_NONE = 0,
  FP8B_KERNEL_GENERIC = 1,      /* SIMT fallback: any block size, unaligned operands */
  FP8B_KERNEL_SKINNY = 2,       /* M <= 48, 16 output columns x all of K per workgroup */
  FP8B_KERNEL_DECODE = 3,       /* M <= 64, 128 columns x a K split per workgroup */
  FP8B_KERNEL_TINY = 4,         /* small grids: 32x32, 32x16 or 64x64 tiles */
  FP8B_KERNEL_PIPE128 = 5,      /* pipelined 128x128 tiles */
  FP8B_KERNEL_PIPE256 = 6,      /* pipelined 256x256 tiles */
  FP8B_KERNEL_PIPE192 = 7,      /* pipelined 192x256 tiles */
  FP8B_KERNEL_PIPE256X128 = 8,  /* pipelined 256x128 tiles */
  FP8B_KERNEL_BS128 = 9,        /* two-stage 128x128 / 256x256 tiles (FP8B_PIPE=0, huge leading dims) */
  FP8B_KERNEL_DECODE_QUANT = 10, /* fp8b_act_quant_matmul, M <= 32: act-quant inside the decode kernel */
  FP8B_KERNEL_SKINNY_QUANT = 11, /* fp8b_act_quant_matmul, M <= 8: act-quant inside the skinny kernel */
  FP8B_KERNEL_TINY_QUANT = 12    /* fp8b_act_quant_matmul, M <= 8 (16 on short K): act-quant inside the small-grid kernel */
} fp8b_kernel;

/* What fp8b_w8a8_block_matmul launches for one call. */
typedef struct fp8b_plan_info {
  int kernel;              /* fp8b_kernel of the main launch                     */
  int tile_m, tile_n;      /* its output tile (rows of A x rows of B)            */
  int splits;              /* K splits; > 1: fp32 partials + split-K sum launch  */
  int kb_per_split;        /* 128-wide K-blocks per split                        */
  int waves;               /* 64-lane waves per workgroup                        */
  int ring;                /* FP8B_KERNEL_DECODE(_QUANT): LDS stages (else 0)    */
  int64_t workgroups;      /* workgroups of the main launch, all splits          */
  int tail_kernel;         /* kernel of the grid's last partial wave, or NONE    */
  int tail_tile_m, tail_tile_n;
  int64_t tail_workgroups;
  int reduce;              /* 1 when the split-K sum kernel follows              */
  size_t workspace_bytes;  /* bytes of fp32 split-K partials (0 when unsplit)     */
  int cu_count;            /* CUs the plan was made for                          */
} fp8b_plan_info;

/*
 * The launches fp8b_w8a8_block_matmul makes for an M x N x K problem with
 * contiguous, 16-byte aligned A and B and K-contiguous scale rows, on a
 * device with cu_count CUs (cu_count <= 0: the current device's). Makes no
 * GPU call when cu_count > 0. Plays the role of the reference's AOT
 * heuristic tables (finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/
 * _helion_aot_fp8_cuda_sm100.py:13-28, which pick a tile config by M);
 * no entry point of the reference reports them.
 */
int fp8b_gemm_plan(int64_t M, int64_t N, int64_t K, int64_t block_n, int64_t block_k,
                   int cu_count, fp8b_plan_info* plan);

/* Name of an fp8b_kernel code ("gemm_pipe256_kernel", ...; "unknown"). */
const char* fp8b_kernel_name(int kernel);

/*
 * fp8b_w8a8_block_matmul without a workspace: it allocates nothing, for
 * callers that cannot call hipMalloc (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation). No counterpart in the
 * reference. Same arguments, semantics and result bits as
 * fp8b_w8a8_block_matmul, minus (workspace, workspace_bytes): the split-K
 * partials go to a library-owned device array of FP8B_NOALLOC_SCRATCH_BYTES,
 * one per GPU, held until the process ends. Shapes whose partials need more
 * (fp8b_gemm_workspace_size() above the limit) return FP8B_ERR_WORKSPACE;
 * on a 256-CU device no plan does (split grids stay within about one wave
 * of workgroups: at most 16 MiB of partials for 128x128 tiles, 32 MiB for
 * 256x128 tiles, under 16 MiB for the split-K decode kernel's 64-row or
 * smaller tiles).
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other threads) race and must be serialised by the caller.
 * The stream must belong to the current device.
 */
#define FP8B_NOALLOC_SCRATCH_BYTES (32u << 20)
int fp8b_w8a8_block_matmul_noalloc(const void* A, int64_t lda,
                                   const void* B, int64_t ldb,
                                   const float* As, int64_t as_sm, int64_t as_sk,
                                   const float* Bs, int64_t bs_sn, int64_t bs_sk,
                                   void* C, int64_t ldc, int out_dtype,
                                   int64_t M, int64_t N, int64_t K,
                                   int64_t block_n, int64_t block_k,
                                   void* stream);

/*
 * Act-quant fused with the block GEMM: C = w8a8(act_quant(x)) against B/Bs
 * with block_n = block_k = 128, with the result bits of fp8b_act_quant
 * (group 128) into (q, s) followed by fp8b_w8a8_block_matmul(q, B, s, Bs).
 * No single counterpart in the reference: it composes the quantiser above
 * with the Helion kernel of
 * finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/fp8.py:19-39 (the
 * act-quant-into-the-GEMM step for small M). On decode plans with M <= 32
 * and skinny or small-grid plans with M <= 8 (small grids: M <= 16 with at
 * most 4 K-blocks per wave) (fp8b_act_quant_matmul_plan
 * reports FP8B_KERNEL_DECODE_QUANT / _SKINNY_QUANT / _TINY_QUANT), with x 16-byte
 * aligned and ldx % 8 == 0, one GEMM kernel reads the bf16 rows and
 * quantises them itself (plus the split-K sum when the plan splits K);
 * otherwise two launches on `stream`: the quantiser writes (q, s) into the
 * workspace, then the GEMM reads them.
 * x : bf16 [M,K] row stride ldx (K % 128 == 0); B, Bs, C as in
 * fp8b_w8a8_block_matmul. workspace: fp8b_act_quant_matmul_workspace_size()
 * bytes, 256-byte aligned.
 */
int fp8b_act_quant_matmul(const void* x, int64_t ldx,
                          const void* B, int64_t ldb,
                          const float* Bs, int64_t bs_sn, int64_t bs_sk,
                          void* C, int64_t ldc, int out_dtype,
                          int64_t M, int64_t N, int64_t K,
                          void* workspace, size_t workspace_bytes,
                          void* stream);

/* Bytes of device workspace fp8b_act_quant_matmul needs for these sizes. */
size_t fp8b_act_quant_matmul_workspace_size(int64_t M, int64_t N, int64_t K);

/*
 * The GEMM launch fp8b_act_quant_matmul makes for an M x N x K problem with a
 * contiguous, 16-byte aligned x (cu_count <= 0: the current device's CUs;
 * no GPU call when cu_count > 0): FP8B_KERNEL_DECODE_QUANT (with its split),
 * FP8B_KERNEL_SKINNY_QUANT or FP8B_KERNEL_TINY_QUANT when one kernel
 * quantises and multiplies,
 * else the plan of the GEMM that
 * follows the act-quant launch (as fp8b_gemm_plan). workspace_bytes is
 * fp8b_act_quant_matmul_workspace_size(). No counterpart in the reference
 * (a plan query like fp8b_gemm_plan).
 */
int fp8b_act_quant_matmul_plan(int64_t M, int64_t N, int64_t K, int cu_count,
                               fp8b_plan_info* plan);

/*
 * Offline 128x128 weight-block quantiser (the format of FP8 checkpoints:
 * e4m3fn weights with one fp32 scale per 128x128 block, "weight_scale_inv"):
 *   Bs[nb,kb] = max(amax over block (nb,kb), 1e-10) / 448   (IEEE)
 *   Wq[n,k]   = float8_e4m3fn(W[n,k] / Bs[n/128,k/128])     (IEEE, RNE)
 * Elements past N or K do not take part; a NaN makes its block's scale NaN
 * and every element of the block 0x7F; otherwise a +-inf makes the block's
 * scale +inf, its +-inf elements 0x7F and its finite elements a signed zero
 * (the act-quant policy above). No counterpart in the reference: it
 * produces the (B, Bs) operands its callers build with torch
 * (scripts/rebench_llm.py:128-131 uses random fp8 instead).
 * W : w_dtype (FP8B_F32 or FP8B_BF16) [N,K] row stride ldw;
 * q : e4m3fn [N,K] row stride ldq (even); Bs (nb,kb) at s[nb*s_sn + kb*s_sk].
 */
int fp8b_weight_quant(const void* W, int64_t ldw, int w_dtype,
                      void* q, int64_t ldq,
                      float* s, int64_t s_sn, int64_t s_sk,
                      int64_t N, int64_t K, void* stream);

/*
 * Gated SiLU: out[m,j] = bf16( bf16(silu(fp32 x[m,j])) * x[m,d+j] ), j < d,
 * for bf16 x [M,2d] (row stride ldx) and out [M,d] (row stride ldo).
 * Replaces _silu_and_mul of
 * activation-helion/activation-helion/torch-ext/activation_helion/act.py:20-28
 * (the SiLU(gate)*up step between the two GEMMs of an FP8 MLP).
 */
int fp8b_silu_and_mul(const void* x, int64_t ldx, void* out, int64_t ldo,
                      int64_t M, int64_t d, void* stream);

/*
 * silu_and_mul for x and out of any of FP8B_F32, FP8B_BF16, FP8B_F16 (the
 * reference kernel is dtype-generic, act.py:20-28):
 *   out[m,j] = TO( TX( TX(silu(fp32 x[m,j])) * x[m,d+j] ) )
 * with TX the type of x and TO that of out, each rounding to nearest even
 * (silu.to(b.dtype) * b in b's dtype, then .to(out.dtype)). bf16 in and out
 * is fp8b_silu_and_mul.
 */
int fp8b_silu_and_mul_typed(const void* x, int64_t ldx, int x_dtype,
                            void* out, int64_t ldo, int out_dtype,
                            int64_t M, int64_t d, void* stream);

/*
 * silu_and_mul fused with per-token-group fp8 quantisation of its result:
 * q/s as fp8b_act_quant would produce from the bf16 output of
 * fp8b_silu_and_mul, without writing that bf16 tensor to memory.
 * No single counterpart in the reference: it composes act.py:20-28 with the
 * quantiser above.
 */
int fp8b_silu_and_mul_quant(const void* x, int64_t ldx,
                            void* q, int64_t ldq,
                            float* s, int64_t s_stride_m, int64_t s_stride_g,
                            int64_t M, int64_t d, int64_t group,
                            void* stream);

/*
 * Gate/up GEMM of a gated FP8 MLP with SiLU(gate)*up and the group-128
 * quantisation of its result in the GEMM epilogue:
 *   h = bf16(w8a8 GEMM of A [M,K] with B [2I,K])   (as fp8b_w8a8_block_matmul)
 *   q, s = act-quant(silu_and_mul(h)) with group 128
 * bit for bit, without writing h. B and Bs must hold the gate and up
 * weights interleaved in 128-row blocks: rows 256t..256t+127 of B are gate
 * rows 128t..128t+127 and rows 256t+128..256t+255 the matching up rows;
 * Bs block row 2t is gate block row t and 2t+1 up block row t.
 * A, As: as fp8b_w8a8_block_matmul (block_n = block_k = 128, A and B
 * 16-byte aligned with lda, ldb multiples of 16, scales of any strides);
 * q: e4m3fn [M,I] row stride ldq (a multiple of 8); scale of (m, g) at
 * s[m*s_stride_m + g*s_stride_g]. Needs I % 128 == 0 and K % 128 == 0.
 * No single counterpart in the reference: it composes the gate/up call of
 * w8a8_block_fp8_matmul (finegrained-fp8-helion/.../fp8.py:28-38) with
 * act.py:20-28 and the quantiser above, as fp8b_silu_and_mul_quant does.
 */
int fp8b_gate_up_silu_quant(const void* A, int64_t lda,
                            const void* B, int64_t ldb,
                            const float* As, int64_t as_sm, int64_t as_sk,
                            const float* Bs, int64_t bs_sn, int64_t bs_sk,
                            void* q, int64_t ldq,
                            float* s, int64_t s_stride_m, int64_t s_stride_g,
                            int64_t M, int64_t I, int64_t K,
                            void* stream);

/*
 * The launch fp8b_gate_up_silu_quant makes for M x I x K on a device with
 * cu_count CUs (cu_count <= 0: the current device's): one unsplit grid of
 * 192x256 or 256x256 tiles (FP8B_KERNEL_PIPE192 / FP8B_KERNEL_PIPE256).
 * Makes no GPU call when cu_count > 0. No counterpart in the reference.
 */
int fp8b_gate_up_plan(int64_t M, int64_t I, int64_t K, int cu_count, fp8b_plan_info* plan);

#ifdef __cplusplus
}
#endif

#endif /* FP8_BLOCKWISE_H */
