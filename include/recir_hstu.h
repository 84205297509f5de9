/*
 * C ABI of the MI355X (gfx950) HSTU jagged attention forward and backward.
 *
 * One shared library, plain pointers and sizes, no C++ or torch types.  Every entry point that
 * launches work does so asynchronously on the HIP stream the caller passes; nothing synchronises
 * with the host, nothing is allocated, and the sequence offsets are read on the device.
 *
 * Operator computed (per sequence b with tokens [s, e), n = e - s, t = num_targets[b],
 * cap = n - t, local positions m, j in [0, n), head h):
 *
 *   keep(m,j)  = (m == j) or (m >= j and j < cap) or contextual(j)                 [causal]
 *   with max_attn_len A > 0 (semi-local, kjt_split_per_feature.cpp:654-668), i = min(m, cap):
 *   keep(m,j)  = (m == j) or (j < i and (i - j <= A or (full_attn_size F > 0 and i >= cap - F)))
 *                or contextual(j)
 *   S(m,j)     = alpha * sum_d q[s+m,h,d] * k[s+j,h,d]  (+ rab[h, m - j + max_seq_len - 1])
 *   P(m,j)     = S * sigmoid(S) * scale          scale = attn_scale or 1 / max_seq_len
 *   out[s+m,h] = sum_j keep(m,j) * P(m,j) * v[s+j,h]
 *   out[r]     = 0 for r >= seq_offsets[B]
 */
#ifndef RECIR_HSTU_H_
#define RECIR_HSTU_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RECIR_HSTU_ABI_VERSION 6

/* element types of q/k (v and out follow: bf16 for BF16 and FP8_E4M3, fp32 for FP32, fp16 for FP16) */
#define RECIR_HSTU_DTYPE_BF16 0
#define RECIR_HSTU_DTYPE_FP32 1
#define RECIR_HSTU_DTYPE_FP8_E4M3 2 /* q,k are OCP e4m3fn bytes with per-head scales; v,out bf16 */
#define RECIR_HSTU_DTYPE_FP16 3     /* IEEE half */

/*
 * Which kernels run a call (recir_hstu_last_kernel names the one that did):
 *   - the kernels written for head dim 128 ("tiled_d128_*", "bwd_tiled_d128_*"): bf16 (forward also
 *     fp8 q/k), Dqk = Dv = 128, 16-byte aligned tensors, the causal or semi-local mask, alpha != 0
 *     when there is a bias;
 *   - the general MFMA kernels ("mfma_*", "bwd_mfma_*"): bf16 or fp16 with Dqk and Dv up to 256,
 *     fp32 up to 128 (fp32 MFMAs, a sixteenth of the bf16 rate); Dqk and Dv independent of each
 *     other, every mask, any alpha; in bf16 1.4 to 1.9 times the time of the first group at its own
 *     shape.  Where every row of every tensor starts at a multiple of 16 bytes (16-byte aligned
 *     tensors, head dims multiples of 8, fp32: 4) rows move in aligned 16-byte pieces; otherwise
 *     (head dims like 25 or 50, a tensor that starts in the middle of a row of a larger one) in
 *     pieces aligned to the element only ("*_elems"), at 1.2 to 1.8 times the time;
 *   - the generic kernels ("generic_*", "bwd_generic_*"): one wave per (token, head), bf16, fp16 or
 *     fp32, any head dim up to 512; one to two orders of magnitude slower.  What is left to them:
 *     head dims above 256 (fp32: 128).
 */

/* flags */
#define RECIR_HSTU_FLAG_OFFSETS_I32 0x1u          /* seq_offsets / num_targets are int32, not int64 */
#define RECIR_HSTU_FLAG_CTX_REFERENCE 0x2u        /* contextual rule of the reference C++ fallback:
                                                     when contextual_seq_len > 0 the keys whose
                                                     target-clamped id is 0 are visible to all
                                                     (kjt_split_per_feature.cpp:672-674).  Default
                                                     rule: keys j < contextual_seq_len visible. */
#define RECIR_HSTU_FLAG_SCALE_PER_TOKEN 0x4u      /* attn_scale is [T], indexed by the query token */
#define RECIR_HSTU_FLAG_REUSE_PLAN 0x8u           /* workspace still holds the work list a previous
                                                     call built for the same seq_offsets, T, B and
                                                     kernel variant: skip rebuilding it (the layers
                                                     of one model step share their offsets)        */
#define RECIR_HSTU_FLAG_GROUPED_LISTS 0x10000u    /* walk each XCD's work list by groups of eight
                                                     (sequence, head) pairs instead of all pairs at
                                                     once (L2 locality against balance).  The library
                                                     chooses this by itself when the tensors of a call
                                                     exceed the last-level cache; the flag forces it
                                                     (tests, tuning).  No effect on results.          */
#define RECIR_HSTU_FLAG_MASK_NONCAUSAL 0x20000u   /* the mask the reference builds for any
                                                     invalid_attn_mask_type other than
                                                     "lower_triangular" (kjt_split_per_feature.cpp:
                                                     650-660): absolute distance of the target-clamped
                                                     ids within max_attn_len, either way round (the
                                                     diagonal alone when max_attn_len is 0), the rows
                                                     of full_attn_size and the contextual keys as in
                                                     the causal case.  General MFMA kernels or
                                                     generic kernels; forward and backward.          */
#define RECIR_HSTU_FLAG_TILED_ONLY 0x40000u       /* reject (RECIR_HSTU_ERR_UNSUPPORTED, with the reason
                                                     in recir_hstu_last_error) a call that only the
                                                     generic kernels cover instead of running it
                                                     there: head dims that exceed 256 (fp32: 128).
                                                     Forward and backward.                           */
#define RECIR_HSTU_FLAG_KERNEL_SHIFT 8            /* bits 8..15: kernel selector for tests/tuning  */
#define RECIR_HSTU_FLAG_KERNEL_MASK 0xff00u       /* 0 auto, 1 generic, 2 general MFMA, 3 head dim 128 */

/* status codes: 0 ok, negative = rejected before any launch, positive = hipError_t of a launch */
#define RECIR_HSTU_OK 0
#define RECIR_HSTU_ERR_INVALID_ARGUMENT (-1)
#define RECIR_HSTU_ERR_UNSUPPORTED (-2)
#define RECIR_HSTU_ERR_WORKSPACE (-3)

/*
 * HSTU jagged attention forward.
 *
 * Replaces: facebook::recir::raggedAttention, the implementation behind the operator schema
 *   hammer::triton_ragged_attention_fwd(int N, float alpha, Tensor q, Tensor k, Tensor v,
 *       Tensor seq_offsets, str invalid_attn_mask_type, Tensor? num_targets, Tensor? attn_scale,
 *       int max_attn_len, int contextual_seq_len, int full_attn_size, int num_softmax_heads)
 *   (recir/ops/kjt_split_per_feature.cpp:602-693, schema :780-783), and the packed accelerator
 *   kernel entry pallas_jagged_hstu_attention (recir/ops/pallas/jagged_hstu_attention.py:1518-1591)
 *   / hstu_ragged_attention_fwd_jax_fn (recir/ops/helion/jagged_hstu_attention.py:830-872).
 *   The causal ("lower_triangular") mask with num_softmax_heads = 0 is covered, plain or
 *   semi-local (max_attn_len, full_attn_size), and the mask of any other invalid_attn_mask_type
 *   string (RECIR_HSTU_FLAG_MASK_NONCAUSAL); the host wrapper rejects softmax heads.
 *
 * q, k          device, [T, H, Dqk] row-major contiguous, element type `dtype`
 * v, out        device, [T, H, Dv]; out is written in full: rows < seq_offsets[B] get the result,
 *               rows in [seq_offsets[B], T) are zeroed (pallas/jagged_hstu_attention.py:323-344)
 * seq_offsets   device, [B+1] int64 (int32 with FLAG_OFFSETS_I32), non-decreasing, last <= T.
 *               Malformed entries are clamped on the device (no fault, result unspecified).
 * num_targets   device, [B] or NULL (= zeros)
 * rab           device float [H, 2*max_seq_len-1] or NULL.  No counterpart in the reference.  A pair
 *               whose m - j falls outside the table (possible only in a sequence longer than
 *               max_seq_len, which is out of contract) gets no bias and adds nothing to drab.
 * attn_scale    device float scalar, [T] with FLAG_SCALE_PER_TOKEN, or NULL (= 1/max_seq_len)
 * q_scale,k_scale  device float [H]; FP8_E4M3 only (dequantisation factors), else NULL
 * max_attn_len, full_attn_size   >= 0; 0, 0 is the plain causal mask; full_attn_size is ignored
 *               when max_attn_len is 0 (as in the reference)
 * workspace     device scratch of at least recir_hstu_attn_fwd_workspace_bytes(...) bytes, 16-byte
 *               aligned; contents need not be initialised; must not be shared by calls that can
 *               overlap on the device
 * hip_stream    hipStream_t (NULL = the null stream)
 */
int recir_hstu_attn_fwd(const void* q, const void* k, const void* v, void* out,
                        const void* seq_offsets, const void* num_targets, const float* rab,
                        const float* attn_scale, const float* q_scale, const float* k_scale,
                        int32_t T, int32_t B, int32_t H, int32_t Dqk, int32_t Dv,
                        int32_t max_seq_len, int32_t contextual_seq_len, int32_t max_attn_len,
                        int32_t full_attn_size, float alpha, int32_t dtype, uint32_t flags,
                        void* workspace, size_t workspace_bytes, void* hip_stream);

/*
 * recir_hstu_attn_fwd for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  Same arguments and results as recir_hstu_attn_fwd without the workspace: the work
 * lists live in a device array of RECIR_HSTU_NOALLOC_SCRATCH_BYTES bytes that is part of the
 * library image (each GPU the library runs on holds its own copy until the process ends).  The
 * call allocates and frees nothing.  Sizes whose work lists do not fit
 * (recir_hstu_attn_fwd_workspace_bytes(...) > RECIR_HSTU_NOALLOC_SCRATCH_BYTES) are rejected with
 * RECIR_HSTU_ERR_WORKSPACE; RECIR_HSTU_FLAG_REUSE_PLAN is rejected (the array is shared by every
 * call on the GPU, so a later call cannot know whose lists it holds).  The device of `hip_stream`
 * must be the current device.  All calls on one GPU share that GPU's array: calls that can overlap
 * on the device (different streams) race and must be ordered by the caller.
 */
#define RECIR_HSTU_NOALLOC_SCRATCH_BYTES (4u << 20)
int recir_hstu_attn_fwd_noalloc(const void* q, const void* k, const void* v, void* out,
                                const void* seq_offsets, const void* num_targets, const float* rab,
                                const float* attn_scale, const float* q_scale, const float* k_scale,
                                int32_t T, int32_t B, int32_t H, int32_t Dqk, int32_t Dv,
                                int32_t max_seq_len, int32_t contextual_seq_len,
                                int32_t max_attn_len, int32_t full_attn_size, float alpha,
                                int32_t dtype, uint32_t flags, void* hip_stream);

/* Scratch size recir_hstu_attn_fwd needs for these sizes (upper bound over all kernel variants). */
size_t recir_hstu_attn_fwd_workspace_bytes(int32_t T, int32_t B, int32_t H, int32_t Dqk,
                                           int32_t Dv, int32_t dtype);

/*
 * HSTU jagged attention backward: gradients of recir_hstu_attn_fwd with respect to q, k and v.
 *
 * Replaces: hstu_ragged_attention_bwd_jax_fn (recir/ops/helion/jagged_hstu_attention.py:875-920,
 *   kernels :356-570, formulas :16-27) and pallas_jagged_hstu_attention_backward with its dQ and
 *   fused dK/dV kernels (recir/ops/pallas/jagged_hstu_attention.py:724-1339); the numerical
 *   definition is autograd through the forward (helion/jagged_hstu_attention.py:260-280).
 *
 *   dP = dO V^T,  dV = P^T dO,  dS = dP keep scale silu'(S),  dQ = alpha dS K,  dK = alpha dS^T Q
 *
 * dout          device, [T, H, Dv], the gradient of the forward's out; rows >= seq_offsets[B] ignored
 * q, k, v       the forward's inputs (bf16, fp16 or fp32; FP8_E4M3 is not supported)
 * dq, dk        device, [T, H, Dqk]; dv device, [T, H, Dv]; same element type as q; written in full
 *               (rows >= seq_offsets[B] zeroed, recir/ops/helion/jagged_hstu_attention.py:916-920)
 * rab           enters S as in the forward
 * drab          device float [H, 2*max_seq_len-1] or NULL: gradient of rab (needs rab),
 *               drab[h, i] = sum of dS(m, j) over the kept pairs of all sequences with
 *               m - j + max_seq_len - 1 == i.  Written in full.  The MFMA kernels (those written
 *               for head dim 128 and the general ones) sum in fixed point (one power-of-two scale
 *               per head, from the head's largest |dout| and the call's largest |v|; integer
 *               additions, so the result is the same bit for bit whatever the order of the
 *               workgroups, like dq, dk and dv); the generic kernels (head dims above 256) add
 *               floats atomically and may differ in the last bits from run to run.  No counterpart
 *               in the reference (which has no rab).  No gradient is produced for attn_scale.
 * attn_scale, flags, sizes, workspace, hip_stream: as for the forward; workspace of at least
 *               recir_hstu_attn_bwd_workspace_bytes(...) bytes, plus, with drab,
 *               recir_hstu_attn_bwd_rab_grad_workspace_bytes(H, max_seq_len)
 */
int recir_hstu_attn_bwd(const void* dout, const void* q, const void* k, const void* v, void* dq,
                        void* dk, void* dv, float* drab, const void* seq_offsets, const void* num_targets,
                        const float* rab, const float* attn_scale, int32_t T, int32_t B, int32_t H,
                        int32_t Dqk, int32_t Dv, int32_t max_seq_len, int32_t contextual_seq_len,
                        int32_t max_attn_len, int32_t full_attn_size, float alpha, int32_t dtype,
                        uint32_t flags, void* workspace, size_t workspace_bytes, void* hip_stream);

/* Additional scratch recir_hstu_attn_bwd needs when drab is requested (the fixed-point table of the
 * sums along the diagonals and the per-head maxima of dout), appended to the scratch below. */
size_t recir_hstu_attn_bwd_rab_grad_workspace_bytes(int32_t H, int32_t max_seq_len);

/* Scratch size recir_hstu_attn_bwd needs for these sizes. */
size_t recir_hstu_attn_bwd_workspace_bytes(int32_t T, int32_t B, int32_t H, int32_t Dqk,
                                           int32_t Dv, int32_t dtype);

/*
 * Per-head symmetric fp8 quantisation of a packed bf16 [T,H,D] tensor:
 *   scale[h] = max(max_{r,d} |x[r,h,d]|, 1e-12) / 448,  codes = e4m3fn(clamp(x / scale[h], +-448)).
 * Replaces: quantizeFp8Rowwise (recir/ops/kjt_split_per_feature.cpp:493-502), applied per head
 * instead of per row.  `scale` ([H] float, device) is both an output and the scratch of the amax
 * reduction.
 */
int recir_hstu_quantize_e4m3_per_head(const void* x_bf16, void* codes_u8, float* scale, int32_t T,
                                      int32_t H, int32_t D, void* hip_stream);

/*
 * The same for a packed tensor whose rows at and after seq_offsets[B] are padding: those rows do
 * not enter the per-head maxima (whatever they hold: the attention kernels ignore and zero them,
 * and so must the scales) and get zero codes.  seq_offsets: device, [B+1], int64 or int32 with
 * RECIR_HSTU_FLAG_OFFSETS_I32; read on the device.
 */
int recir_hstu_quantize_e4m3_per_head_rows(const void* x_bf16, void* codes_u8, float* scale, int32_t T,
                                           int32_t H, int32_t D, const void* seq_offsets, int32_t B,
                                           uint32_t flags, void* hip_stream);

/*
 * Measurement aid, no counterpart in the reference: a plain device-to-device copy of `bytes` bytes
 * (multiple of 16, both pointers 16-byte aligned) by one kernel.  Hardware counters that are read
 * for the attention kernel (FETCH_SIZE, WRITE_SIZE) are scaled by what they read for this copy,
 * whose traffic is known exactly.
 */
int recir_hstu_calibration_copy(void* dst, const void* src, size_t bytes, void* hip_stream);

/*
 * Measurement aid, no counterpart in the reference: stand-alone loops with the instruction mix of the
 * tiled forward kernel and none of its bookkeeping, to price that kernel against what the chip
 * sustains rather than against the data-sheet peak alone.
 *   kind 0  bf16 MFMAs only (v_mfma_f32_32x32x16_bf16 back to back, operands in registers)
 *   kind 1  the forward's tile loop, plain arrangement: per 32-row x 64-key wave tile 32 MFMAs, SiLU of
 *           32 scores per lane, 48 LDS fragment reads, 8 global -> LDS copies, one barrier
 *   kind 2  the same work in the skewed arrangement of the forward's leading unmasked tiles
 *   kind 3  kind 2 with 64 query rows per wave, one workgroup (256 rows) per CU, one wave per SIMD: every
 *           LDS fragment feeds two MFMAs (a design the attention kernels do not use; priced here).  A
 *           workgroup does twice the work: FLOPs = workgroups * tiles * 4 * 64 * 32768
 * pieces (kinds 1, 2) removes parts, timing only: 1 no SiLU, 2 no LDS fragment reads, 12 no copies and
 * no barrier, 14 MFMAs + SiLU only; 0 keeps everything (kind 3: 0 or 2).
 * k, v: device, [rows, 4, 128] bf16, read as `sequences` runs of rows / 64 / sequences key tiles;
 * q: device, at least [128, 4, 128] bf16.  What they hold is the caller's choice (random values or
 * zeros: the clock the chip grants depends on the operands).  `workgroups` workgroups of 256 threads
 * (two fit a CU) each run `tiles` (even) key tiles: FLOPs = workgroups * tiles * 4 * 32 * 32768.
 * stats: device, [workgroups][4] uint64: shader-clock cycles and 100 MHz ticks of one wave's loop, then
 * the loop's start and end on the 100 MHz counter (one time base for all workgroups of a launch).
 * sink: device, [workgroups * 256] float, written once at the end.
 */
int recir_hstu_calibration_mfma_loop(int32_t kind, int32_t pieces, const void* k, const void* v, const void* q,
                                     size_t rows, int32_t sequences, int32_t tiles, int32_t workgroups, float alpha,
                                     uint64_t* stats, float* sink, void* hip_stream);

/* Thread-local, NUL-terminated description of the last non-zero status on this thread. */
const char* recir_hstu_last_error(void);

/* RECIR_HSTU_ABI_VERSION the library was built with. */
int recir_hstu_abi_version(void);

/* Name of the kernel variant the last successful recir_hstu_attn_fwd on this thread launched. */
const char* recir_hstu_last_kernel(void);

#ifdef __cplusplus
}
#endif
#endif /* RECIR_HSTU_H_ */
