/*
 * mqk.h -- C ABI of the MI355X (gfx950) fused QKV projection + QK-Norm + RoPE
 * library (libmqk.so).
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream passed
 * as `void*` (a hipStream_t; NULL = the default stream).  bf16 tensors are
 * passed as `mqk_bf16*` (the raw 16-bit pattern).  All tensors are dense and
 * row-major ("contiguous" in PyTorch terms).  Calls are asynchronous on the
 * given stream, never synchronize, never allocate device memory, and may be
 * made from any host thread.  Kernels launch on the calling thread's current
 * HIP device: every pointer, the workspace and the stream must belong to it
 * (a process driving several GPUs calls hipSetDevice first).  Return value:
 * MQK_OK (0) or a negative mqk error code; mqk_error_string() turns it into
 * text and mqk_last_error_detail() names the argument or HIP error involved
 * (per host thread).
 *
 * Reference interface each entry point replaces (mini-qwen-llm):
 *   mqk_fused_qkv_rope_bf16   <- fused_qkv_rope()      mini_qwen/kernels/fused_qkv_rope.py:130-195
 *   mqk_fused_qkv_rope_f32    <- fused_qkv_rope() called with fp32 tensors (same lines)
 *   mqk_fused_qkv_rope_f16    <- fused_qkv_rope() called with fp16 tensors (same lines)
 *   mqk_qk_norm_rope_bf16     <- _qk_norm_rope_kernel  mini_qwen/kernels/fused_qkv_rope.py:46-127
 *   mqk_w4a16_gemm(_ex)       <- w4a16_gemm()          mini_qwen/kernels/w4a16_gemm.py:194-247
 *   mqk_fused_qkv_rope_w4a16  <- the W4A16 attention front (3x LinearW4A16 + RMSNorm + RoPE),
 *                                mini_qwen/model/layers/attention.py:102-109 (prefill), :136-148 (decode)
 *   mqk_fused_qkv_rope_paged_* <- the above + the paged KV-cache scatter, write_kv_decode /
 *                                _write_kv_cache_kernel (mini_qwen/kernels/paged_attn_prefill.py:27-56, :232-254)
 *   mqk_fused_qkv_rope_ex_*    <- the above + varlen (cu_seqlens) positions (paged_attn_prefill.py:188-199)
 *                                and the decoder layer's input RMSNorm (qwen3.py:58-59, rms_norm.py:11-18)
 */
#ifndef MQK_H_
#define MQK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t mqk_bf16;
typedef uint16_t mqk_f16;  /* IEEE half */

enum mqk_status {
  MQK_OK = 0,
  MQK_ERR_NULL_POINTER = -1,     /* a required pointer is NULL */
  MQK_ERR_BAD_SHAPE = -2,        /* a size is negative, zero where it must not be, or inconsistent */
  MQK_ERR_UNSUPPORTED = -3,      /* a valid shape this library does not implement (e.g. head_dim 66) */
  MQK_ERR_MISALIGNED = -4,       /* a pointer is not 16-byte aligned */
  MQK_ERR_WORKSPACE = -5,        /* workspace NULL or smaller than mqk_*_workspace_size() */
  MQK_ERR_HIP = -6,              /* a HIP runtime call failed (launch, attribute query) */
  MQK_ERR_BAD_OPTION = -7        /* unknown option name or value out of range */
};

/* Scale element type of the W4A16 entry points. */
enum mqk_scale_type { MQK_SCALE_BF16 = 0, MQK_SCALE_FP16 = 1 };

/* Library version, major*10000 + minor*100 + patch. */
int mqk_version(void);
const char* mqk_error_string(int status);
/* Detail of the last error raised on the calling host thread ("" if none). */
const char* mqk_last_error_detail(void);

/*
 * Fused Q/K/V projection + per-head RMSNorm of Q and K + rotate-half RoPE of
 * Q and K; V is the plain projection.  Replaces fused_qkv_rope()
 * (mini_qwen/kernels/fused_qkv_rope.py:130-195; frozen signature :24-35).
 *
 *   x        [T, hidden]          T = B*S tokens
 *   w_q      [Hq*D, hidden]       nn.Linear layout (out_features, in_features)
 *   w_k, w_v [Hkv*D, hidden]
 *   q_gamma, k_gamma [D]          QK-Norm weights, shared by all heads
 *   cos, sin [cos_rows, D]        row stride D
 *   positions [T] int32 or NULL   NULL: prefill mode, token t uses row t % S
 *                                 (fused_qkv_rope.py:109); otherwise row
 *                                 positions[t] (:107).  Rows outside
 *                                 [0, cos_rows) are clamped into range (the
 *                                 reference reads out of bounds there).
 *   q [T, Hq, D], k [T, Hkv, D], v [T, Hkv, D]   outputs, bf16
 *   eps                           RMSNorm epsilon (the reference hard-codes 1e-6, :187)
 *   workspace/ws_bytes            device scratch of at least
 *                                 mqk_fused_qkv_rope_workspace_size(T, Hq, Hkv, hidden)
 *                                 bytes.  It must be zero-filled once when
 *                                 first allocated (it holds arrival counters
 *                                 that every call leaves at zero again).  One
 *                                 workspace must not be used by two calls that
 *                                 may overlap (same or different streams).
 *
 * Supported: D == 128, or D == 64 with Hq and Hkv even (the kernels run
 * 128-column blocks of two heads; the reference's default Qwen3Config has
 * head_dim 64, mini_qwen/config.py:13), hidden % 64 == 0, Hq >= 1, Hkv >= 1,
 * T >= 0 (T == 0 is
 * a no-op), x/w/q/k/v 16-byte aligned.  Numerics: bf16 inputs, fp32
 * accumulation on MFMA, the norm and RoPE are applied to the fp32 accumulator
 * (the projection is not rounded to bf16 before the norm), one bf16 rounding
 * per output.
 * Other head sizes that are a multiple of 8 up to 512 (e.g. 80, 96, 192, 256) run
 * as the reference composes the op (fused_qkv_rope.py:166-190): the projections
 * into q / k / v (rounded to bf16; one launch of the fused plan with q and k
 * stored as projected where Hq * D and Hkv * D are whole 128-column blocks, else
 * one or more launches per projection), then one QK-Norm + RoPE launch in place
 * on q and k (which also writes the paged-cache rows).  Size the workspace with
 * mqk_fused_qkv_rope_workspace_size_hd (a smaller one runs the tile kernels);
 * k / v must be given even with a paged cache.
 */
int mqk_fused_qkv_rope_bf16(const mqk_bf16* x, const mqk_bf16* w_q, const mqk_bf16* w_k,
                            const mqk_bf16* w_v, const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                            const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                            int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                            int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                            void* workspace, size_t ws_bytes, void* stream);

/*
 * fp32 twin of mqk_fused_qkv_rope_bf16: x, weights, q_gamma / k_gamma and the
 * cos / sin tables are fp32, and q / k / v are written in fp32
 * (fused_qkv_rope() called with fp32 tensors, mini_qwen/kernels/fused_qkv_rope.py:130-195).
 * Products and sums in fp32 on the matrix cores; norm and RoPE in fp32; one
 * rounding per output, to fp32.  Deliberate difference: the reference's Triton
 * kernel rounds Q and K to bf16 before storing them into its fp32 outputs
 * (:117-120); this entry point keeps fp32 precision (it computes the fp32
 * composition of the unfused path).  Same position rules and validation as the
 * bf16 entry point; hidden must be a multiple of 32.  Needs no workspace.
 * Launches on `stream` without synchronising.
 */
int mqk_fused_qkv_rope_f32(const float* x, const float* w_q, const float* w_k, const float* w_v,
                           const float* q_gamma, const float* k_gamma, const float* cos, const float* sin,
                           const int32_t* positions, int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv,
                           int D, int64_t cos_rows, float eps, float* q, float* k, float* v, void* stream);

/*
 * fp16 twin of mqk_fused_qkv_rope_f32 (the reference op on fp16 tensors, e.g. a
 * model loaded with dtype=float16, mini_qwen/model/loader.py:12-52): every
 * float input fp16, q / k / v written in fp16.  The fp32 front's kernel with
 * fp16 tiles on the fp16 matrix cores (exact products, fp32 sums); norm and
 * RoPE in fp32; one fp16 rounding per output.  Deliberate differences: the
 * reference rounds the fp16 GEMM output before the norm (:167-169) and Q / K to
 * bf16 before the fp16 store (:117-120); neither rounding happens here.  Same
 * validation; no workspace.
 */
int mqk_fused_qkv_rope_f16(const mqk_f16* x, const mqk_f16* w_q, const mqk_f16* w_k, const mqk_f16* w_v,
                           const mqk_f16* q_gamma, const mqk_f16* k_gamma, const mqk_f16* cos, const mqk_f16* sin,
                           const int32_t* positions, int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv,
                           int D, int64_t cos_rows, float eps, mqk_f16* q, mqk_f16* k, mqk_f16* v, void* stream);

/* Workspace bytes needed by mqk_fused_qkv_rope_bf16 / _w4a16 for these sizes
 * (0 when the chosen kernels need none; pair tiles need 66 KiB per pair of
 * 256-row workgroups, e.g. 16.9 MB for BASELINE config 4, 33 KiB per pair of
 * 128-row ones, e.g. 4.3 MB for Qwen3-8B at T = 1024).  Hq and Hkv are counted in 128-column
 * blocks: the head counts for D == 128, Hq / 2 and Hkv / 2 for D == 64.  The
 * same holds for mqk_fused_qkv_rope_ex_workspace_size. */
size_t mqk_fused_qkv_rope_workspace_size(int64_t T, int Hq, int Hkv, int64_t hidden);

/* Workspace bytes for any supported head_dim, with Hq and Hkv the head counts.
 * For head_dim 128 and 64 it equals mqk_fused_qkv_rope_workspace_size over
 * 128-column blocks.  Other head sizes whose q and k / v widths (Hq * head_dim,
 * Hkv * head_dim) are whole 128-column blocks run the three projections as one
 * launch of the fused op's plan over those blocks (decode kernel, decode
 * blocks, split-K, single-head or pair tiles), q and k stored as projected,
 * then the norm + RoPE launch; otherwise each projection of whole blocks is
 * planned on its own, and the rest run on the tile kernels (W4A16 up to 16
 * rows: the column-parallel kernel).  Each runs its planned form when the
 * workspace holds what that plan needs, and the tile kernels otherwise; this
 * returns the most they need, for either weight format, with or without the
 * fused input RMSNorm (which, for W4A16 weights at these head sizes, needs the
 * one-launch form: whole 128-column widths).  Like the reference's
 * op, which infers D from the norm weight
 * (mini_qwen/kernels/fused_qkv_rope.py:155-160), the entry points take any head
 * size; the reference sizes no workspace, so this query has no counterpart
 * there.  For the _ex entry points take the larger of this and
 * mqk_fused_qkv_rope_ex_workspace_size. */
size_t mqk_fused_qkv_rope_workspace_size_hd(int64_t T, int Hq, int Hkv, int64_t hidden, int head_dim);

/*
 * mqk_fused_qkv_rope_bf16 without a workspace argument: allocates nothing, for
 * callers that cannot call hipMalloc (code under HIP-graph capture, tight
 * serving loops, harnesses that forbid allocation).  It has no counterpart in
 * the reference.  The decode kernel's counters and partials live in a fixed
 * device array of 68.25 KiB + 8 MiB per GPU, held until the process ends; calls
 * whose decode launch needs more (e.g. T <= 64 with more than 256 heads x
 * splits) return MQK_ERR_WORKSPACE before launching anything, and larger T run
 * with fewer 64-row blocks per decode launch (bit-identical results).  Every
 * call on a GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller.
 */
int mqk_fused_qkv_rope_bf16_noalloc(const mqk_bf16* x, const mqk_bf16* w_q, const mqk_bf16* w_k,
                                    const mqk_bf16* w_v, const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                                    const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                                    int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                                    int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                                    void* stream);

/*
 * QK-Norm + RoPE alone on already-projected q/k (bf16), the functional twin
 * of _qk_norm_rope_kernel (mini_qwen/kernels/fused_qkv_rope.py:46-127):
 *   q_raw [T, Hq, D] -> q_out, k_raw [T, Hkv, D] -> k_out.
 * Position rules as above.  Either projection may be skipped by passing Hq or
 * Hkv == 0.  In-place (q_out == q_raw) is allowed.
 */
int mqk_qk_norm_rope_bf16(const mqk_bf16* q_raw, const mqk_bf16* k_raw, const mqk_bf16* q_gamma,
                          const mqk_bf16* k_gamma, const mqk_bf16* cos, const mqk_bf16* sin,
                          const int32_t* positions, int64_t T, int64_t S, int Hq, int Hkv, int D,
                          int64_t cos_rows, float eps, mqk_bf16* q_out, mqk_bf16* k_out,
                          void* stream);

/*
 * W4A16 GEMM, out[M, N] = x[M, K] @ dequant(qweight)   (w4a16_gemm.py:194-247)
 *   qweight [K/8, N] int32   nibble i of qweight[j, n] is W[8j+i, n] (w4a16_gemm.py:11)
 *   scales  [K/group, N]     bf16 or fp16 (scale_type)
 *   qzeros  [K/group, N/8]   int32, packed along N, nibble i of qzeros[g, j] is z[g, 8j+i]
 *   dequant: (q - z) * s computed exactly in fp32; M <= 16 multiplies the exact
 *   fp32 weight with fp32 sums (column-parallel kernels, no workspace), larger M
 *   rounds it once to bf16 for the bf16 MFMA tiles.
 * Supported: K % 64 == 0, group % 64 == 0, K % group == 0, N % 8 == 0.
 */
int mqk_w4a16_gemm(const mqk_bf16* x, const int32_t* qweight, const void* scales,
                   const int32_t* qzeros, int64_t M, int64_t K, int64_t N, int group,
                   int scale_type, mqk_bf16* out, void* stream);

/* Workspace bytes mqk_w4a16_gemm_ex needs for these sizes (0: none). */
size_t mqk_w4a16_gemm_workspace_size(int64_t M, int64_t K, int64_t N);

/*
 * mqk_w4a16_gemm with the kernel choice of the fused op: M <= 16 (the decode
 * regime of w4a16_gemm.py:110-189, the reference's M = 1 GEMV, and its published
 * decode shapes M in {1, 4, 8, 16}, K = 1024, N = 4096) runs the column-parallel
 * kernels of mqk_w4a16_gemm (no workspace); mid M runs on the split-K decode
 * kernel, which streams the packed weights over every CU once for up to sixteen
 * 64-row blocks; larger M on the tile kernels.  The workspace is
 * as for mqk_fused_qkv_rope_bf16 (zero-filled once at allocation, not shared by
 * calls that may overlap).  N not a multiple of 128 or operands not 16-byte
 * aligned: the tile kernels of mqk_w4a16_gemm, no workspace needed.
 */
int mqk_w4a16_gemm_ex(const mqk_bf16* x, const int32_t* qweight, const void* scales, const int32_t* qzeros,
                      int64_t M, int64_t K, int64_t N, int group, int scale_type, mqk_bf16* out,
                      void* workspace, size_t ws_bytes, void* stream);

/*
 * Fused W4A16 front: three int4 projections (q, k, v; each in the
 * mqk_w4a16_gemm layout with N = Hq*D, Hkv*D, Hkv*D) + QK-Norm + RoPE,
 * with the same position rules, outputs and workspace as
 * mqk_fused_qkv_rope_bf16 (head sizes other than 64 and 128, multiples of 8 up
 * to 512, as there: three mqk_w4a16_gemm launches into q / k / v, then the
 * in-place QK-Norm + RoPE; no input RMSNorm at those sizes).  Replaces attention.py:102-109 / :136-148, where
 * the reference runs w4a16_gemm x3 then an unfused RMSNorm and RoPE.
 */
int mqk_fused_qkv_rope_w4a16(const mqk_bf16* x, const int32_t* qw_q, const void* sc_q,
                             const int32_t* qz_q, const int32_t* qw_k, const void* sc_k,
                             const int32_t* qz_k, const int32_t* qw_v, const void* sc_v,
                             const int32_t* qz_v, int group, int scale_type,
                             const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                             const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                             int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                             int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                             void* workspace, size_t ws_bytes, void* stream);

/*
 * Paged KV cache destination of the fused ops below: K and V rows are also written
 * into the caches of mini_qwen/cache/kv_cache.py:3-6 (both [num_blocks, block_size,
 * Hkv, D] bf16).  Token t belongs to sequence kv_seq[t] (NULL: t / S) at position
 * kv_pos[t] (NULL: t % S) and lands in block block_table[seq * bt_cols + pos /
 * block_size], slot pos % block_size -- the addressing of the reference's
 * _write_kv_cache_kernel (mini_qwen/kernels/paged_attn_prefill.py:27-56).  Entries
 * whose sequence, page or block falls outside the given table are skipped.
 */
typedef struct mqk_paged_kv {
  mqk_bf16* k_cache;            /* [num_blocks, block_size, Hkv, D], 16-byte aligned */
  mqk_bf16* v_cache;
  const int32_t* block_table;   /* [bt_rows, bt_cols] int32 */
  int64_t bt_rows;
  int64_t bt_cols;
  int64_t num_blocks;
  int32_t block_size;           /* the reference fixes 16 */
  const int32_t* kv_seq;        /* [T] or NULL (required when positions != NULL) */
  const int32_t* kv_pos;        /* [T] or NULL (required when positions != NULL) */
} mqk_paged_kv;

/*
 * mqk_fused_qkv_rope_bf16 / _w4a16 that also write K and V into a paged KV cache,
 * fusing the reference's separate scatter (write_kv_decode, paged_attn_prefill.py
 * :232-254, and the scatter at :203-213) into the projection epilogue.  k and v
 * may be NULL to write the cache only (the decode step, whose attention reads
 * the cache).  Everything else as the unpaged entry points.
 */
int mqk_fused_qkv_rope_paged_bf16(const mqk_bf16* x, const mqk_bf16* w_q, const mqk_bf16* w_k,
                                  const mqk_bf16* w_v, const mqk_bf16* q_gamma,
                                  const mqk_bf16* k_gamma, const mqk_bf16* cos, const mqk_bf16* sin,
                                  const int32_t* positions, int64_t T, int64_t S, int64_t hidden,
                                  int Hq, int Hkv, int D, int64_t cos_rows, float eps, mqk_bf16* q,
                                  mqk_bf16* k, mqk_bf16* v, const mqk_paged_kv* kv, void* workspace,
                                  size_t ws_bytes, void* stream);

int mqk_fused_qkv_rope_paged_w4a16(const mqk_bf16* x, const int32_t* qw_q, const void* sc_q,
                                   const int32_t* qz_q, const int32_t* qw_k, const void* sc_k,
                                   const int32_t* qz_k, const int32_t* qw_v, const void* sc_v,
                                   const int32_t* qz_v, int group, int scale_type,
                                   const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                                   const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                                   int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                                   int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                                   const mqk_paged_kv* kv, void* workspace, size_t ws_bytes,
                                   void* stream);

/*
 * Optional features of the extended entry points below.  Zero-fill the struct and
 * set what is used; an all-zero struct (or ext == NULL) gives the plain op.
 *
 * Varlen prefill (cu_seqlens != NULL; `positions` must then be NULL): the T
 * tokens are n_seqs packed sequences, token t belonging to sequence s with
 * cu_seqlens[s] <= t < cu_seqlens[s+1].  Its RoPE row, and its position in the
 * paged KV cache, is t - cu_seqlens[s] + (seq_pos0 ? seq_pos0[s] : 0), and its
 * block_table row is s -- the batch_ids / positions that paged_attn_prefill
 * derives from cu_seqlens (mini_qwen/kernels/paged_attn_prefill.py:188-199).
 * This lifts fused_qkv_rope's equal-length restriction (row t % S,
 * fused_qkv_rope.py:109), so one call serves a whole continuous batch.
 * cu_seqlens lives in device memory and is not read by the host: offsets that
 * are not non-decreasing from 0 to T give unspecified rows (clamped into the
 * table, never read or written out of bounds).
 *
 * Input RMSNorm (in_gamma != NULL): the projection input is
 * in_gamma * bf16(x_fp32 * rsqrt(mean(x^2) + in_eps)), rounded to bf16 -- the
 * decoder layer's input_layernorm (mini_qwen/model/layers/rms_norm.py:11-18,
 * applied at mini_qwen/model/qwen3.py:58-59) computed inside the op, so the
 * normalised activations never go to HBM.  The per-token scale is computed by a
 * pre-pass into the workspace: size it with mqk_fused_qkv_rope_ex_workspace_size.
 *
 * kv != NULL: the paged KV-cache write of mqk_fused_qkv_rope_paged_* (in
 * varlen mode kv_seq / kv_pos may be NULL: the sequence and position above).
 */
typedef struct mqk_fused_ext {
  const int32_t* cu_seqlens;    /* [n_seqs + 1] int32, device memory, or NULL */
  const int32_t* seq_pos0;      /* [n_seqs] position of each sequence's first token, or NULL (0) */
  int64_t n_seqs;
  const mqk_bf16* in_gamma;     /* [hidden] input RMSNorm weight, or NULL */
  float in_eps;
  const mqk_paged_kv* kv;       /* paged KV cache, or NULL */
} mqk_fused_ext;

/* Workspace bytes needed by the _ex entry points (the plain size plus the
 * input-norm scales when ext->in_gamma is set). */
size_t mqk_fused_qkv_rope_ex_workspace_size(int64_t T, int Hq, int Hkv, int64_t hidden,
                                            const mqk_fused_ext* ext);

/* mqk_fused_qkv_rope_bf16 / _w4a16 with the features of `ext` (NULL: none).  With
 * ext->kv set, k and v may be NULL (cache only). */
int mqk_fused_qkv_rope_ex_bf16(const mqk_bf16* x, const mqk_bf16* w_q, const mqk_bf16* w_k,
                               const mqk_bf16* w_v, const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                               const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                               int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                               int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                               const mqk_fused_ext* ext, void* workspace, size_t ws_bytes, void* stream);

int mqk_fused_qkv_rope_ex_w4a16(const mqk_bf16* x, const int32_t* qw_q, const void* sc_q,
                                const int32_t* qz_q, const int32_t* qw_k, const void* sc_k,
                                const int32_t* qz_k, const int32_t* qw_v, const void* sc_v,
                                const int32_t* qz_v, int group, int scale_type,
                                const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                                const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                                int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                                int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                                const mqk_fused_ext* ext, void* workspace, size_t ws_bytes,
                                void* stream);

/*
 * Process-wide tuning knobs (used by benchmarks and tests; defaults are
 * chosen by shape).  Names:
 *   "prefill_tile"   0 = auto, otherwise a tile variant id (see mqk_tile_variants)
 *   "decode_max_t"   largest T routed to the split-K decode kernel (0..64, default 64;
 *                    0 disables it)
 *   "decode_splits"  0 = auto, otherwise the split-K factor of the decode kernel (1..16,
 *                    at most 32 64-wide k tiles per split, 13 when a launch covers several
 *                    64-row blocks; otherwise the tile kernel runs)
 *   "group_m"        row tiles per tile-ordering group of the tile kernel (default 8)
 *   "tail_split"     1 (default): when the last, partial row tile of a prefill holds at most 64
 *                    rows and would cost a whole extra round of tiles over the CUs, those rows
 *                    run on the split-K decode kernel in a second launch; 0: never
 *   "decode_blocks"  16 (default): most 64-row blocks of split-K decode launches one call
 *                    with 64 < T tokens may run as (instead of a tile launch whose few tiles
 *                    leave most CUs idle), used where a cost model of both paths says the
 *                    launches are faster; 0: never
 *   "decode_passes"  16 (default): most 64-row blocks one decode launch covers, streaming
 *                    the weights once for all of them (1..16; the workspace size grows with it)
 *   "decode_cost_model"  1 (default): decode blocks run where the cost model prefers them
 *                    to a tile launch; 0: whenever decode_blocks allows (for measurements)
 *   "decode_max_spins"  polls (~64 ns apart) a decode launch of several blocks makes while
 *                    a block's designated finisher waits for its last splits, before it
 *                    hands the block to the last split to arrive (default 16384, ~1 ms;
 *                    0 hands off at once; for tests of the hand-off).  The split-K tile
 *                    launch bounds each split's wait for the others the same way.
 *   "decode_force_recompute"  1: the decode kernel and the split-K tile launch take their
 *                    recompute path (used when the splits of a head or tile ran on more than one XCD) for every
 *                    head / tile; for tests
 *   "tile_ksplit"    bf16 calls with fewer tiles than CUs (64 < T up to ~1000 tokens at
 *                    hidden 4096): 1 (default) = a split-K tile launch (each tile's K range
 *                    over several workgroups of one XCD, fp32 partials in the workspace)
 *                    where a cost model prefers it to the decode blocks and the plain tile
 *                    launch; 0 = never; 2..16 = that split count whenever a split launch fits
 *   "head_tiles"     1 (default): bf16 calls whose single-head tiles (64 x 128, else
 *                    128 x 128) fill at most one round over the CUs run as one such tile
 *                    launch where the cost model prefers it to the decode blocks and the
 *                    split-K tile launch; 0: never
 *   "pair_tiles"     1 (default): bf16 calls with head_dim 128 may run as pair tiles (two
 *                    256-row workgroups per 3 heads, 256 x 192 each, variant 24, or per 5
 *                    heads, 256 x 320 each, variant 25; 128-row forms 26 and 27, a 192-row
 *                    form 28; the two
 *                    share one head whose RMSNorm sums they exchange through the
 *                    workspace) where the planner prefers them (e.g. BASELINE config 4:
 *                    512 tiles in two rounds instead of 640 of 256 x 256; Qwen3-8B at
 *                    T = 768 .. 1024: one round of 128-row pairs instead of split-K
 *                    tiles); 0: never
 *   "pair_max_spins" polls (~1 us apart) a pair tile makes for its partner's sums before it
 *                    hands its half of the shared head over (default 16384; for tests)
 *   "pair_hold"      (tests) side 1 of every pair waits this many ~4 us intervals before
 *                    publishing its sums, so that side 0 takes the hand-over path (default 0)
 *   "pair_cross_xcd" (tests) 1: the two sides of a pair take adjacent workgroup ids, which
 *                    the round-robin dispatch places on different XCDs (default 0: one XCD)
 * Returns MQK_OK or MQK_ERR_BAD_OPTION.  mqk_get_option also reads "device_cus" and
 * "device_xcds": the compute units and XCDs of the current device, as the planner and
 * the decode kernel's grid use them (hipDeviceGetAttribute; -1 for unknown names).
 * Heads the decode kernel (and tiles the split-K tile launch) finished on their
 * recompute path are counted in the first word after the per-head counters of the
 * workspace (byte offset 4096).
 */
int mqk_set_option(const char* name, int64_t value);
int64_t mqk_get_option(const char* name);
/* Human-readable list of tile variants, "id:BMxBN/waves;...". */
const char* mqk_tile_variants(void);

/*
 * Measurement probe, no counterpart in the reference: reads `bytes` bytes at the
 * device pointer src (16-byte aligned, bytes % 16 == 0) once, with 16-byte
 * non-temporal loads over `blocks` workgroups of 512 threads, and writes one
 * 32-bit word per workgroup to out[blocks].  bench.py times it as the HBM read
 * ceiling of the decode step's weight stream.  Launches on `stream`.
 */
int mqk_read_probe(const void* src, size_t bytes, int blocks, uint32_t* out, void* stream);

/*
 * Measurement probe, no counterpart in the reference: one lane runs a dependent
 * chain of `spins` fp32 FMAs and writes to the device array out[3] the shader
 * clock cycles (s_memtime) and 100 MHz ticks (s_memrealtime) that passed over
 * it, and the chain's result; out[0] / out[1] * 100 is the shader clock in MHz
 * while it ran.  bench.py reads it right after a timed region.
 */
int mqk_clock_probe(uint64_t* out, int spins, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MQK_H_ */
