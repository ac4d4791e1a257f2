/*
 * rwkv_hip.h — C ABI of the MI355X (gfx950) WKV-7 + .rwkvq hot path.
 *
 * Drop-in replacement for the MLX/Metal kernel dispatch of SwiftRWKV's
 * RWKVKernel and RWKVQuant modules.  Each entry point names the Swift
 * function (RafaelUI/SwiftRWKV, file:line) whose kernel launch it replaces.
 *
 * Conventions
 *  - Plain C, no C++ or torch types.  All tensors are caller-allocated device
 *    buffers (HIP device pointers), row-major, densely packed.
 *  - Shapes: WKV inputs [B,T,H,64]; state [B,H,64(dv),64(dk)] (value index =
 *    row, key index = column); train checkpoints [B,H,T/16,64,64].
 *  - A NULL `h_in` / `d_h_out` means an all-zero state / cotangent (the
 *    reference's `hIn: nil`, `MLXArray.zeros`).
 *  - Every call takes a `hipStream_t` (passed as void*; NULL = default stream)
 *    and is asynchronous on it.  Nothing allocates device memory.
 *  - Errors come back as rwkv_status instead of the reference's
 *    precondition traps; rwkv_last_error() holds a message (thread-local).
 *  - "applies" predicates return 1/0 exactly like the reference's
 *    *Applies functions, so a caller falls back the same way.
 *  - Launch counters mirror the reference's test counters
 *    (wkv7SequenceLaunches, wkv7TrainForwardLaunches, rwkvq*Calls).
 */
#ifndef RWKV_HIP_H
#define RWKV_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RWKV_HIP_ABI_VERSION 1

typedef enum {
    RWKV_OK = 0,
    RWKV_E_SHAPE = 1,        /* shape precondition violated (T, D, OUT, IN, rows ...) */
    RWKV_E_DTYPE = 2,        /* unsupported dtype code */
    RWKV_E_UNSUPPORTED = 3,  /* valid request this library does not implement */
    RWKV_E_FORMAT = 4,       /* malformed .rwkvq / safetensors container or manifest */
    RWKV_E_HIP = 5,          /* HIP runtime error (launch, device) */
    RWKV_E_NULL = 6,         /* required pointer is NULL */
    RWKV_E_IO = 7            /* file missing / unreadable */
} rwkv_status;

typedef enum { RWKV_F32 = 0, RWKV_BF16 = 1, RWKV_F16 = 2 } rwkv_dtype;

/* Library identity and error reporting. */
int rwkv_abi_version(void);
const char* rwkv_status_string(rwkv_status s);
const char* rwkv_last_error(void);

/* WKV7_HEAD_SIZE / WKV7_CHUNK — Sources/RWKVKernel/WKV7.swift:7-8. */
int rwkv_wkv7_head_size(void);
int rwkv_wkv7_chunk(void);

/* ───────────────────────────── RWKVKernel: WKV-7 ───────────────────────────── */

/* Whole-sequence frozen forward, any T >= 1, one launch.
 * Replaces wkv7SequenceForward (Sources/RWKVKernel/WKV7.swift:242-264).
 * r..b: [B,T,H,64] of in_dt (widened to fp32 in registers, exactly like the
 * reference's asType(.float32)); h_in [B,H,64,64] fp32 or NULL;
 * out [B,T,H,64] fp32; h_out [B,H,64,64] fp32. */
rwkv_status rwkv_wkv7_seq_fwd(const void* r, const void* w, const void* k, const void* v,
                              const void* a, const void* b, rwkv_dtype in_dt,
                              const float* h_in, float* out, float* h_out,
                              int64_t B, int64_t T, int64_t H, void* stream);

/* Whole-sequence frozen forward computed in 32-token time chunks, in
 * parallel over the chunks (the same recurrence as rwkv_wkv7_seq_fwd,
 * WKV7.swift:213-220, in its chunked matrix form): for sequences with few
 * (batch, head) rows, where one workgroup per row walking T steps leaves the
 * GPU idle.  Same arguments and layouts as rwkv_wkv7_seq_fwd, plus a device
 * workspace of at least rwkv_wkv7_chunked_workspace(B, T, H) bytes, 16-byte
 * aligned (48 KiB per 32 tokens per head).  Agrees with rwkv_wkv7_seq_fwd to
 * fp32 rounding, not bitwise.  h_out may alias h_in.  Prefill counterpart of
 * wkv7SequenceForward (WKV7.swift:242-264); no separate reference entry. */
int64_t rwkv_wkv7_chunked_workspace(int64_t B, int64_t T, int64_t H);
rwkv_status rwkv_wkv7_seq_fwd_chunked(const void* r, const void* w, const void* k, const void* v,
                                      const void* a, const void* b, rwkv_dtype in_dt,
                                      const float* h_in, float* out, float* h_out,
                                      int64_t B, int64_t T, int64_t H,
                                      void* workspace, int64_t workspace_bytes, void* stream);

/* rwkv_wkv7_seq_fwd_chunked with no workspace argument and no allocation:
 * the chunk transforms live in a static 64 MiB device array of the library
 * (one per GPU it runs on, held until the process ends), so at most
 * B·H·ceil(T/32) <= 1365; larger passes return RWKV_E_SHAPE.  No counterpart
 * in the reference: for callers that cannot allocate device memory (code
 * under stream capture, serving loops, hosts that forbid hipMalloc).  Calls
 * on one GPU share the array: calls that overlap on one GPU race.  Nothing
 * in it needs clearing between calls. */
rwkv_status rwkv_wkv7_seq_fwd_chunked_static(const void* r, const void* w, const void* k, const void* v,
                                             const void* a, const void* b, rwkv_dtype in_dt,
                                             const float* h_in, float* out, float* h_out,
                                             int64_t B, int64_t T, int64_t H, void* stream);

/* One 16-token chunk, also emitting sa = S·a per step.
 * Replaces wkv7ChunkForward (WKV7.swift:64-82).  T must equal 16.
 * h_in is required (the reference passes an explicit state). */
rwkv_status rwkv_wkv7_chunk_fwd(const void* r, const void* w, const void* k, const void* v,
                                const void* a, const void* b, rwkv_dtype in_dt,
                                const float* h_in, float* out, float* h_out, float* sa_out,
                                int64_t B, int64_t T, int64_t H, void* stream);

/* Training forward: out, h_out, sa [B,T,H,64] and the state after every
 * 16-token chunk, h_ckpt [B,H,T/16,64,64].  T % 16 == 0.  Bitwise equal to
 * rwkv_wkv7_seq_fwd on out/h_out.  Replaces ckptFwdKernel launched by
 * wkv7TrainWithState (Sources/RWKVKernel/WKV7Train.swift:26-97,390-397). */
rwkv_status rwkv_wkv7_train_fwd(const void* r, const void* w, const void* k, const void* v,
                                const void* a, const void* b, rwkv_dtype in_dt,
                                const float* h_in, float* out, float* h_out,
                                float* sa_out, float* h_ckpt,
                                int64_t B, int64_t T, int64_t H, void* stream);

/* Backward from checkpoints.  Replaces ckptBwdKernelV2 / ckptBwdKernel
 * launched by the VJP of wkv7TrainWithState (WKV7Train.swift:99-339,410-420).
 * h_in: the forward's initial state [B,H,64,64] fp32 or NULL (zeros) — the
 * VJP's primal h0, from which variant 2 recomputes the first chunk's states.
 * h_ckpt, sa: the training forward's outputs.  d_out [B,T,H,64] fp32;
 * d_h_out [B,H,64,64] fp32 or NULL.  Gradients dr..db [B,T,H,64] are written
 * in g_dt (the primal's dtype, :440,462); dh_in [B,H,64,64] fp32.
 * variant: 2 = the default (wkv7BackwardV2 = true; column-owned, states
 * recomputed forward from h_in / the previous checkpoint), 1 = the
 * reference's row-owned ckptBwdKernel (WKV7Train.swift:99-205: one wave per
 * head, states recovered by dividing by w, so the gradients formed from them,
 * dr / dw / da, carry the forward's rounding amplified by up to Π 1/w over a
 * 16-step chunk; h_in unused). */
rwkv_status rwkv_wkv7_train_bwd(const void* r, const void* w, const void* k, const void* v,
                                const void* a, const void* b, rwkv_dtype in_dt,
                                const float* h_in, const float* h_ckpt, const float* sa,
                                const float* d_out, const float* d_h_out,
                                void* dr, void* dw, void* dk, void* dv, void* da, void* db,
                                rwkv_dtype g_dt, float* dh_in,
                                int64_t B, int64_t T, int64_t H, int variant, void* stream);

/* One-token decode step for B rows.  r..b [B,H,64]; h_in/h_out [B,H,64,64]
 * fp32 (may alias: in-place update is safe); out [B,H,64] fp32.
 * Replaces wkv7StepForward (Sources/RWKVKernel/WKV7DecodeKernels.swift:73-89),
 * which is B = 1 only; bitwise equal to rwkv_wkv7_seq_fwd at T = 1. */
rwkv_status rwkv_wkv7_step(const void* r, const void* w, const void* k, const void* v,
                           const void* a, const void* b, rwkv_dtype in_dt,
                           const float* h_in, float* out, float* h_out,
                           int64_t B, int64_t H, void* stream);

/* wkvTailApplies (WKV7DecodeKernels.swift:92): S % 32 == 0. */
int rwkv_wkv_tail_applies(int64_t S);

/* tmix tail over N rows: ((gn(wkv)·lnw + lnb) + Σ(r·k·rk)·v)·g, two-pass
 * group norm per (row, head).  wkv, r, k, v, g, out [N, H·S] fp32;
 * rk, lnw, lnb [H·S] fp32.  Replaces wkvTail (WKV7DecodeKernels.swift:106-178). */
rwkv_status rwkv_wkv_tail(const float* wkv, const float* r, const float* k, const float* v,
                          const float* rk, const float* lnw, const float* lnb, const float* g,
                          float* out, int64_t N, int64_t H, int64_t S, float eps, void* stream);

/* rwkv_wkv_tail with the output in out_dt: f32 (rwkv_wkv_tail) or f16, the
 * rounding the fp16 long pass of the o_proj matmul applies to its input
 * (X070Backbone.swift:337-356 casts x to the fp16 base), so a parallel pass
 * hands the projection the values it would use, in half the bytes.  The same
 * replaced interface: wkvTail (WKV7DecodeKernels.swift:106-178) feeding
 * RWKVBlock's o_proj (RWKVBlock.swift:269-273). */
rwkv_status rwkv_wkv_tail_to(const float* wkv, const float* r, const float* k, const float* v,
                             const float* rk, const float* lnw, const float* lnb, const float* g,
                             void* out, rwkv_dtype out_dt, int64_t N, int64_t H, int64_t S, float eps,
                             void* stream);

/* Decode step and tmix tail in one launch, fp32, head size 64: the state
 * update of rwkv_wkv7_step followed by rwkv_wkv_tail (S = 64) on its output,
 * bitwise equal to calling the two.  No single counterpart in the reference:
 * it replaces the pair wkv7StepForward + wkvTail that X070Generation's tmix
 * step launches back to back (WKV7DecodeKernels.swift:73-89, 106-178), saving
 * one launch per layer and token.  r..b, g, out [B,H,64]; h_in/h_out
 * [B,H,64,64] (may alias; h_in NULL = zeros); rk, lnw, lnb [H·64];
 * wkv_out [B,H,64] receives the step output when non-NULL. */
rwkv_status rwkv_wkv7_step_tail(const float* r, const float* w, const float* k, const float* v,
                                const float* a, const float* b, const float* h_in, float* h_out,
                                const float* rk, const float* lnw, const float* lnb, const float* g,
                                float* wkv_out, float* out, int64_t B, int64_t H, float eps,
                                void* stream);

/* ───────────────────────────── RWKVQuant: dequant / GEMV ───────────────────────────── */

/* sb6 K3 interleave → dense [OUT, IN] in out_dt (combine always in fp32).
 * qblk [OUT, IN/32·(16+4·xbits)] u8; qsqm [OUT, IN/32·2] u8; ddm [OUT, IN/256·2]
 * fp16 bits.  Replaces rwkvqDequantDense (Sources/RWKVQuant/RwkvqDequant.swift:160-183). */
rwkv_status rwkv_sb6_dequant(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                             void* out, rwkv_dtype out_dt, int64_t OUT, int64_t IN, int xbits,
                             void* stream);

/* sym interleave → dense.  bits 8: qblk [OUT, IN] int8 (IN % 16 == 0);
 * bits 6: qblk [OUT, IN/32·24] (IN % 32 == 0).  qs [OUT, IN/16] int8;
 * d [OUT, ceil(IN/256)] fp16 bits.  Replaces rwkvqDequantSym and its
 * off-superblock chain rwkvqDequantSymReference (RwkvqDequant.swift:409-466). */
rwkv_status rwkv_sym_dequant(const uint8_t* qblk, const uint8_t* qs, const uint16_t* d,
                             void* out, rwkv_dtype out_dt, int64_t OUT, int64_t IN, int bits,
                             void* stream);

/* Rows ids[0..n) of a sym matrix, dequantised on demand (the embedding
 * table): out [n, IN] = the rows rwkv_sym_dequant would give for those matrix
 * rows, bitwise.  ids int32 on the device; an id outside [0, OUT) gives a row
 * of NaN; n == 0 is a no-op (ids and out may be NULL).  Replaces RwkvqSymRowTable.rows (Sources/RWKVQuant/RwkvqSymRows.swift:43-53),
 * which takes 8-bit tables; 6-bit ones work as well. */
rwkv_status rwkv_sym_rows(const int32_t* ids, int64_t n, const uint8_t* qblk, const uint8_t* qs,
                          const uint16_t* d, void* out, rwkv_dtype out_dt, int64_t OUT, int64_t IN,
                          int bits, void* stream);

/* rwkvqSb6GEMVApplies (Sources/RWKVQuant/RwkvqSb6GEMV.swift:159-164), same table. */
int rwkv_sb6_gemv_applies(int64_t OUT, int64_t IN, int xbits, int super_block, int64_t rows);

/* y[N, OUT] = x[N, IN] · Wᵀ straight from the K3 bytes, fp32.  N >= 1 rows
 * share one pass over the weights (the reference launches one row at a time);
 * xbsum is computed inside.  Replaces rwkvqSb6GEMV (RwkvqSb6GEMV.swift:170-190). */
rwkv_status rwkv_sb6_gemv(const float* x, int64_t N,
                          const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                          float* y, int64_t OUT, int64_t IN, int xbits, void* stream);

/* Batched sb6 4-bit GEMV on the matrix cores: y[n] = W·x[n] for 2 <= N <= 32
 * input rows with the weights streamed once (bf16 MFMA; the inputs split
 * exactly into three bf16 parts, the block scales folded in fp32 per
 * 32-column unit).  Per row within fp32 rounding of rwkv_sb6_gemv on that
 * row alone (not bitwise).  out_per: rows per input row (OUT for one matrix,
 * D for a row-concatenated fused group reading x [N, OUT/out_per, IN]);
 * multiple of 64.  epilogue as rwkv_sb6_gemv_ep (0 store, 1 add to y,
 * 2 relu²).  workspace: >= rwkv_sb6_gemv_batch_workspace(N, OUT, IN, out_per)
 * bytes, 16-byte aligned (fp32 partial sums of the K slices).  The batched
 * counterpart of rwkvqSb6GEMV (RwkvqSb6GEMV.swift:159-190), which the
 * reference launches once per row (BatchGenerate.swift:58-90). */
int rwkv_sb6_gemv_batch_applies(int64_t N, int64_t OUT, int64_t IN, int xbits, int64_t out_per);
int64_t rwkv_sb6_gemv_batch_workspace(int64_t N, int64_t OUT, int64_t IN, int64_t out_per);
rwkv_status rwkv_sb6_gemv_batch(const float* x, int64_t N, const uint8_t* qblk, const uint8_t* qsqm,
                                const uint16_t* ddm, float* y, int64_t OUT, int64_t IN, int xbits,
                                int64_t out_per, int epilogue, void* workspace, int64_t workspace_bytes,
                                void* stream);

/* The sb6 4-bit weights of rwkv_sb6_gemv_batch in the matrix cores' own
 * order ("T16"; no counterpart in the reference, whose weights stay in K3):
 * per 16-row tile and group of 4 32-column units, the codes as one 1 KiB
 * block (lane-ordered for 16-byte loads, each lane's dwords of the four
 * units together) and the unit scales precomputed: s = half(qs·d) fp16
 * [16 rows][4 units], m = half(qm·dm) as two exact bf16 parts [16 rows]
 * [4 high, 4 low].  tq OUT·IN/2 bytes (16-byte aligned), ts OUT·IN/32 fp16,
 * tm OUT·IN/16 bf16.  OUT % 16 == 0, IN % 256 == 0.  A permutation and the
 * kernels' own rounding of s and m: exact. */
rwkv_status rwkv_sb6_t16_pack(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm, int64_t OUT,
                              int64_t IN, uint8_t* tq, uint16_t* ts, uint16_t* tm, void* stream);

/* rwkv_sb6_gemv_batch over T16 weights (rwkv_sb6_t16_pack): the same shapes,
 * epilogues, workspace and applies rule (xbits 0); the m·Σx term of every
 * unit on the matrix cores as well.  Within fp32 rounding of the K3 batch
 * kernel and of rwkv_sb6_gemv per row (not bitwise).  The batched
 * counterpart of rwkvqSb6GEMV (RwkvqSb6GEMV.swift:159-190). */
rwkv_status rwkv_sb6_gemv_batch_t16(const float* x, int64_t N, const uint8_t* tq, const uint16_t* ts,
                                    const uint16_t* tm, float* y, int64_t OUT, int64_t IN, int64_t out_per,
                                    int epilogue, void* workspace, int64_t workspace_bytes, void* stream);

/* Kernel launches one rwkv_sb6_gemv_batch_t16 call makes: 1 where it takes
 * the row-owned kernel (OUT·K <= 2^24 and K <= 3072; or K <= 4096 with
 * (OUT/16)·ceil(N/16) <= 64 or > 256), 2 (K slices and their reduction)
 * otherwise, 0 where it does not apply.  For launch accounting of
 * captured graphs; no counterpart in the reference. */
int rwkv_sb6_gemv_batch_t16_launches(int64_t N, int64_t OUT, int64_t IN, int64_t out_per);

/* rwkv_sb6_gemv_batch_t16 by the row-owned kernel alone: one workgroup per
 * 16-row tile whose waves split K and sum their partial products in LDS, so
 * one launch and no workspace.  Same shapes, epilogues and accuracy; for
 * matrices of a few million weights, where K slices leave each workgroup a
 * few units of work (rwkv_sb6_gemv_batch_t16 chooses it there itself).  The
 * batched counterpart of rwkvqSb6GEMV (RwkvqSb6GEMV.swift:159-190). */
rwkv_status rwkv_sb6_gemv_batch_t16_rows(const float* x, int64_t N, const uint8_t* tq, const uint16_t* ts,
                                         const uint16_t* tm, float* y, int64_t OUT, int64_t IN, int64_t out_per,
                                         int epilogue, void* stream);

/* sb6 counterpart of the sym r/k/v fusion (no counterpart in the reference,
 * which fuses sym groups only, RwkvqSymGEMV.swift:343-358): K = OUT/out_per
 * row-concatenated sb6 matrices in one launch; row `o` of input row n uses
 * x[n·K + o/out_per]; x holds N·K rows.  Same arithmetic per row as
 * rwkv_sb6_gemv. */
rwkv_status rwkv_sb6_gemv_fused(const float* x, int64_t N,
                                const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                                float* y, int64_t OUT, int64_t IN, int xbits, int64_t out_per,
                                void* stream);

/* rwkvqSymGEMVApplies (Sources/RWKVQuant/RwkvqSymGEMV.swift:213-218), same table. */
int rwkv_sym_gemv_applies(int64_t OUT, int64_t IN, int bits, int64_t rows);

/* sym GEMV.  out_per == OUT: y[N, OUT] = x[N, IN]·Wᵀ (rwkvqSymGEMV, :223-247).
 * out_per < OUT: K = OUT/out_per row-concatenated matrices; row `o` of input
 * row n uses x[n·K + o/out_per] (symGEMVFused, :343-358).  x holds N·K rows. */
rwkv_status rwkv_sym_gemv(const float* x, int64_t N,
                          const uint8_t* qblk, const uint8_t* qs, const uint16_t* d,
                          float* y, int64_t OUT, int64_t IN, int bits, int64_t out_per,
                          void* stream);

/* GEMV with an epilogue: epilogue 0 stores y = x·Wᵀ (rwkv_sb6_gemv /
 * rwkv_sym_gemv with out_per = OUT), 1 adds it to y (the residual updates
 * x = x + pj(·), X070Generation.swift:493-497), 2 stores relu(x·Wᵀ)² (cmixStep's
 * relu(pj(xk)) squared, :308-309).  Same per-row arithmetic as the plain
 * entry points; the epilogue is the separate operations' exact arithmetic. */
rwkv_status rwkv_sb6_gemv_ep(const float* x, int64_t N,
                             const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                             float* y, int64_t OUT, int64_t IN, int xbits, int epilogue,
                             void* stream);
rwkv_status rwkv_sym_gemv_ep(const float* x, int64_t N,
                             const uint8_t* qblk, const uint8_t* qs, const uint16_t* d,
                             float* y, int64_t OUT, int64_t IN, int bits, int epilogue,
                             void* stream);

/* Parallel-pass projection (many input rows) on the matrix cores: the long
 * pass of X070Backbone.baseMatmul with an fp16 base (Sources/RWKVGen/X070Backbone.swift:337-356,
 * 733-739): y = fp16(fp16(x)·fp16(W)ᵀ) where fp16(W) is exactly the dequant
 * rwkv_sb6_dequant(out_dt = f16) stores, products summed in fp32, the sum
 * rounded to fp16 (the fp16 matmul's output) — computed from the K3 bytes
 * without writing the dense weight.  sb6 with 4, 5 or 6-bit codes (xbits
 * 0..2); OUT and out_per multiples of 128, IN of 256 (rwkv_sb6_gemm_applies).
 * x [groups][M][lda] in x_dt (f32 or f16; groups = OUT / out_per, matrix g
 * at x + g·x_group_stride elements): output feature o reads group o / out_per,
 * so r/k/v with their own inputs run as one launch.  y [M][ldy]:
 * epilogue 0 stores, 1 adds into y (fp32; the residual update), 2 stores
 * relu(·)² as fp16 (y is then an fp16 buffer; cmix's key, exact in fp16).
 * workspace: NULL, or device memory of rwkv_quant_gemm_workspace(M, OUT, IN)
 * bytes (16-byte aligned; a smaller one is refused before any launch).  With
 * it, shapes with few 128 × 128 output tiles split the K sum into ranges
 * summed in a fixed order by a second kernel (the same bound, deterministic,
 * far faster for a few hundred rows), and shapes with at least 128 output
 * tiles of 256 × 256 and f16 inputs dequantise the weight into the
 * workspace (rwkv_sb6_dequant / rwkv_sym_dequant, f16) and run rwkv_f16_gemm
 * over it — the same products in the same order, so bitwise the one-range
 * result, at 2-2.5x its speed for M >= 4096.  With NULL the launch is one
 * range.  Launches sharing a workspace must not overlap. */
int rwkv_sb6_gemm_applies(int64_t OUT, int64_t IN, int xbits, int64_t out_per);
int64_t rwkv_quant_gemm_workspace(int64_t M, int64_t OUT, int64_t IN);
rwkv_status rwkv_sb6_gemm(const void* x, rwkv_dtype x_dt, int64_t M, int64_t lda, int64_t x_group_stride,
                          const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm, void* y, int64_t ldy,
                          int64_t OUT, int64_t IN, int xbits, int64_t out_per, int epilogue, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* The same long pass for sym matrices (8-bit codes, or 6-bit in the loader's
 * interleave; qs [OUT, IN/16] int8, d [OUT, IN/256] fp16): fp16(W) is exactly
 * what rwkv_sym_dequant(out_dt = f16) stores (the fp16 branch of
 * rwkvqDequantSym computes in half, RwkvqDequant.swift:350-388), the rest as
 * rwkv_sb6_gemm (arguments, groups, epilogues, workspace, rwkv_sym_gemm_applies). */
int rwkv_sym_gemm_applies(int64_t OUT, int64_t IN, int bits, int64_t out_per);
rwkv_status rwkv_sym_gemm(const void* x, rwkv_dtype x_dt, int64_t M, int64_t lda, int64_t x_group_stride,
                          const uint8_t* qblk, const uint8_t* qs, const uint16_t* d, void* y, int64_t ldy,
                          int64_t OUT, int64_t IN, int bits, int64_t out_per, int epilogue, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* The long pass's fp16 matmul on a dense fp16 weight w [OUT][IN] (K
 * contiguous; the fp16 matmul of baseMatmul once the weight is dequantised,
 * X070Backbone.swift:337-356): y = epilogue(fp16(x·wᵀ)), fp32 sums, x
 * [groups][M][lda] f16 with groups = OUT / out_per as rwkv_sb6_gemm, the same
 * epilogues.  256 × 256 output tiles: OUT and out_per multiples of 256, IN of
 * 128, lda >= IN and a multiple of 8, x and w 16-byte aligned
 * (rwkv_f16_gemm_applies for lda = IN).  Each output is rwkv_sb6_gemm's /
 * rwkv_sym_gemm's bitwise when w is the fp16 weight those decode. */
int rwkv_f16_gemm_applies(int64_t M, int64_t OUT, int64_t IN, int64_t out_per);
rwkv_status rwkv_f16_gemm(const void* x, int64_t M, int64_t lda, int64_t x_group_stride, const void* w, void* y,
                          int64_t ldy, int64_t OUT, int64_t IN, int64_t out_per, int epilogue, void* stream);

/* ───────────────────────── x070 decode step around the hot path ───────────────────────── */
/* fp32 activations; dense vector parameters fp32 (an fp16 file's values
 * widen exactly); low-rank matrices f16 (the reference's `lin` narrowing,
 * X070Generation.swift:248-253: input rounded to fp16, fp32 accumulation,
 * product rounded to fp16) or f32 (plain fp32). */

/* y[n] = LayerNorm(src_n)·w + b over D (layerNorm_, X070Generation.swift:505-515:
 * mean, then mean squared deviation, eps).  src_n = x[n] ([N, D], f32/f16) or,
 * with ids (int32, device), row ids[n] of the table x [rows, D] (embedForBlock
 * + ln0, :489-490); an id outside [0, rows) gives a NaN row.  D % 256 == 0 and
 * D ≤ 4096, or D ∈ {2048, 4096, 8192}; y must not alias x.  N ≤ 65535. */
rwkv_status rwkv_layer_norm(const void* x, rwkv_dtype x_dt, const int32_t* ids, int64_t rows,
                            const float* w, const float* b, float* y, int64_t N, int64_t D,
                            float eps, void* stream);

/* Layer norm + token shift + lerps of tmixStep (:214-239; ln1 of stepEager
 * :492) or cmixStep (:303-308; ln2 :495-496): xl = LN(x[n]); xx = prev[n] − xl;
 * prev[n] ← xl; m_c = xl + xx·coef[c].  nc = 6: coef [6, D] in the order
 * r, k, v, w, a, g; out0 [N, 3, D] ← (m_r, m_k, m_v) (the fused r/k/v GEMV
 * input), out1 [N, 4, D] ← (m_w, m_a, m_v, m_g) (the low-rank inputs).
 * nc = 1: out0 [N, D].  Widths as rwkv_layer_norm; the outputs must not
 * alias x. */
rwkv_status rwkv_x070_shift_mix(const float* x, const float* lnw, const float* lnb, float* prev,
                                const float* coef, int nc, float* out0, float* out1,
                                int64_t N, int64_t D, float eps, void* stream);

/* First layers of the low-rank branches (tmixStep :256-276, the inner lin of
 * each): wcat [rw + ra + rv + rg, D] = w_lora_A ‖ a_lora_A ‖ v_lora_A ‖
 * g_lora_A rows; la [N, rw + ra + rv + rg] = tanh(lin(xw, ·)) ‖ lin(xa, ·) ‖
 * lin(xv, ·) ‖ sigmoid(lin(xg, ·)), xw, xa, xv, xg = rows of xmix [N, 4, D].
 * with_v = 0 (layer 0) skips the v branch. */
rwkv_status rwkv_x070_lora_in(const float* xmix, const void* wcat, rwkv_dtype w_dt, int64_t rw,
                              int64_t ra, int64_t rv, int64_t rg, int with_v, float* la, int64_t N,
                              int64_t D, void* stream);

/* One input row (batch 1): the layer's fused r/k/v GEMV (rwkv_sb6_gemv_fused
 * with N = 1: x_rkv [OUT / out_per, IN] → y_rkv [OUT]) and its low-rank first
 * layers (rwkv_x070_lora_in with N = 1, D = IN) in one launch — tmixStep
 * computes them one after the other (:237-239, :256-276); both depend only on
 * the shift mixes.  The results are bitwise those of the two entries.  4-bit sb6 with
 * fp16 low-rank matrices and the GEMV plans of the x070 shapes take the single
 * launch; other inputs run the two entries.  Counts one sb6_fused and one
 * x070 launch. */
rwkv_status rwkv_x070_rkv_lora(const float* x_rkv, const uint8_t* qblk, const uint8_t* qsqm,
                               const uint16_t* ddm, float* y_rkv, int64_t OUT, int64_t IN, int xbits,
                               int64_t out_per, const float* xmix, const void* wcat, rwkv_dtype w_dt,
                               int64_t rw, int64_t ra, int64_t rv, int64_t rg, int with_v, float* la,
                               void* stream);

/* The tmix core (tmixStep :256-294): second layers of the low-rank branches
 * for each head's rows (w2 [D, rw], a2 [D, ra], v2 [D, rv], g2 [D, rg] in
 * w_dt; biases fp32): w = exp(−0.606531·σ(lin + w2_bias)), a = σ(lin + a2_bias),
 * vv = σ(lin + v2_bias), gate = lin; kk = l2norm(k0·k_k) per head;
 * k = k0·(1 + (a − 1)·k_a); v = layer0 ? v0 (v_first ← v0) : v0 + (v_first − v0)·vv;
 * the WKV step with (r, w, k, v, −kk, kk·a) on state [N, H, 64, 64] in place
 * (rwkv_wkv7_step's arithmetic); out [N, H·64] = the tail
 * ((GroupNorm(y)·lnx_w + lnx_b + Σ(r·k·r_k)·v)·gate, rwkv_wkv_tail's).
 * y_rkv [N, 3·H·64] = r | k0 | v0 (the fused r/k/v GEMV output); la from
 * rwkv_x070_lora_in.  shift_src / shift_dst (both or neither): copies the
 * row shift_src [N, H·64] to shift_dst, the token-shift state that
 * rwkv_x070_rkv_lora_ln read (its LN row, for the next token). */
rwkv_status rwkv_x070_tmix_core(const float* y_rkv, const float* la, const void* w2, const void* a2,
                                const void* v2, const void* g2, rwkv_dtype w_dt, int64_t rw,
                                int64_t ra, int64_t rv, int64_t rg, const float* w2_bias,
                                const float* a2_bias, const float* v2_bias, const float* k_k,
                                const float* k_a, const float* r_k, const float* lnx_w,
                                const float* lnx_b, float* v_first, int layer0, float* state,
                                float* out, int64_t N, int64_t H, float eps, const float* shift_src,
                                float* shift_dst, void* stream);

/* ─────── one-row decode launches that form their GEMV inputs themselves ───────
 * (no counterpart in the reference, whose step runs the layer norm, the token
 * shift and the lerps as separate ops, X070Generation.swift :214-239,
 * :303-308): each GEMV workgroup forms its input row — LN(x) with (ln_w,
 * ln_b), then the lerp LN(x) + (prev − LN(x))·coef — in rwkv_x070_shift_mix's
 * exact arithmetic, so a step built from them is bitwise the one built from
 * shift_mix + the GEMV entries, with two launches per layer fewer.  `prev`
 * (the token-shift state) is read, not written: LN(x) goes to `xln`, and a
 * later launch of the same layer (rwkv_x070_tmix_core / rwkv_x070_ffn_value
 * with shift_src = xln) stores it as the next `prev`, after every reader of
 * the old one has run.  Batch 1, 4-bit sb6, the x070 plans (D ≤ 4096):
 * rwkv_x070_ln_fused_applies(D, F, xbits). */
int rwkv_x070_ln_fused_applies(int64_t D, int64_t F, int xbits);
/* rwkv_x070_rkv_lora with its inputs formed from x [D]: coef6 [6, D] in the
 * order r, k, v, w, a, g (rwkv_x070_shift_mix's); fp16 low-rank matrices. */
rwkv_status rwkv_x070_rkv_lora_ln(const float* x, const float* ln_w, const float* ln_b, const float* prev,
                                  const float* coef6, float eps, float* xln, const uint8_t* qblk,
                                  const uint8_t* qsqm, const uint16_t* ddm, float* y_rkv, int64_t D,
                                  int xbits, const void* wcat, rwkv_dtype w_dt, int64_t rw, int64_t ra,
                                  int64_t rv, int64_t rg, int with_v, float* la, void* stream);
/* The ffn key GEMV with the relu² epilogue (cmixStep :308-309): hk [F] =
 * relu(W_key · (LN2(x) + (prev − LN2(x))·coef))², coef [D]. */
rwkv_status rwkv_x070_ffn_key_ln(const float* x, const float* ln_w, const float* ln_b, const float* prev,
                                 const float* coef, float eps, float* xln, const uint8_t* qblk,
                                 const uint8_t* qsqm, const uint16_t* ddm, float* hk, int64_t F, int64_t D,
                                 int xbits, void* stream);
/* The ffn value GEMV with the residual add (x [D] += W_value · hk [F],
 * :309 / :496), and with shift_src / shift_dst (both or neither) the copy
 * shift_dst [D] ← shift_src [D]. */
rwkv_status rwkv_x070_ffn_value(const float* hk, const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                                float* x, int64_t D, int64_t F, int xbits, const float* shift_src,
                                float* shift_dst, void* stream);

/* ───────────────────────── x070 parallel (prefill) pass ───────────────────────── */
/* B rows of T tokens flattened as n = b·T + t; lengths (int32, device) [B]
 * gives each row's real tokens (right padding; NULL = all T). */

/* Token shift over a sequence with its lerps (rwkvTokenShift and the x_c
 * lerps of rwkvTmixForward / rwkvCmixForward, Sources/RWKVGen/RWKVBlock.swift:145-183,
 * 300-307): for layer-normed rows xl [B·T, D], prev_t = xl[n − 1] (t > 0) or
 * prev_in[b] (the carried shift state; NULL = zeros); m_c = xl + (prev_t − xl)·coef[c].
 * Coefficients [0, n0) → y0 (f32 or f16; element (n, c) at n·y0_row + c·y0_coef);
 * y1 (f32, may be NULL) receives the coefficients [y1_first, nc) at n·y1_row + c·y1_coef (the
 * low-rank branches read v, w, a, g: y1_first = 2 leaves r and k to y0 alone); prev_out [B, D] ← xl
 * of each row's last real token (gatherLast, :320-335).  nc = 6 (r, k, v, w, a, g) or 1.
 * prev_out may alias prev_in (the carried state of a row is updated in place;
 * a row with lengths[b] = 0 keeps it). */
rwkv_status rwkv_x070_seq_shift_mix(const float* xl, const float* prev_in, float* prev_out, const int32_t* lengths,
                                    const float* coef, int nc, int n0, void* y0, rwkv_dtype y0_dt, int64_t y0_row,
                                    int64_t y0_coef, float* y1, int64_t y1_row, int64_t y1_coef, int y1_first, int64_t B, int64_t T,
                                    int64_t D, void* stream);

/* The time-mix arithmetic between the projections and the recurrence
 * (rwkvTmixForward, RWKVBlock.swift:185-237): y_rkv [B·T, 3D] = r | k0 | v0,
 * low-rank second layers ww, aa, vv [B·T, D] before their biases (vv NULL at
 * layer 0) → the WKV-7 inputs r, w, k, v, a, b [B·T, D] (w = exp(−0.606531·σ(ww + w_bias)),
 * a = −kk, b = kk·σ(aa + a_bias), kk = l2norm(k0·k_k) per head,
 * k = k0·(1 + (σ(aa + a_bias) − 1)·k_a), v mixed with v_first [B·T, D] or, at
 * layer 0, written to it), pad steps neutral (w = 1, k = 0, b = 0,
 * :232-237), and k_bonus = k unmasked for the tail. */
/* The low-rank w / a / v / g branches of the parallel pass (rwkvTmixForward,
 * Sources/RWKVGen/RWKVBlock.swift:185-226) for M rows: ww = tanh(x_w·A_wᵀ)·B_wᵀ,
 * aa = (x_a·A_aᵀ)·B_aᵀ, vv = (x_v·A_vᵀ)·B_vᵀ (with_v; layer 0 has no v branch),
 * gate = sigmoid(x_g·A_gᵀ)·B_gᵀ, in fp32 on the matrix cores (matrices f16 or
 * f32, widened exactly; no fp16 narrowing on this path).  mix [6, M, D] fp32:
 * the lerped rows in rwkv_x070_seq_shift_mix's coefficient order (r, k, v, w,
 * a, g); wcat [rw + ra + rv + rg, D]: A_w, A_a, A_v, A_g stacked; w2 / a2 / v2 /
 * g2 [D, rank]; la [M, rw + ra + rv + rg] fp32 holds the inner products.
 * Ranks multiples of 16, D of 16.  Long passes (M·D above 2^21) with f16
 * matrices, ranks and D multiples of 32 (rwkv_x070_seq_lora_split) carry
 * each fp32 activation as two fp16 parts, hi = fp16(x) and lo = fp16(x − hi),
 * on the fp16 matrix cores: every product is exact in fp32 and the sums are
 * fp32, the activation enters with 22 of its 24 significant bits (error at
 * most 2^-22·|x|, 2^-25 absolute below fp16's normal range); activations
 * must stay below 65504 in magnitude. */
rwkv_status rwkv_x070_seq_lora(const float* mix, int64_t M, int64_t D, const void* wcat, const void* w2,
                               const void* a2, const void* v2, const void* g2, rwkv_dtype w_dt, int64_t rw,
                               int64_t ra, int64_t rv, int64_t rg, int with_v, float* la, float* ww, float* aa,
                               float* vv, float* gate, void* stream);
/* Whether rwkv_x070_seq_lora takes the two-part fp16 kernel for this pass. */
int rwkv_x070_seq_lora_split(int64_t M, int64_t D, rwkv_dtype w_dt, int64_t rw, int64_t ra, int64_t rv, int64_t rg);
rwkv_status rwkv_x070_seq_tmix_pre(const float* y_rkv, const float* ww, const float* aa, const float* vv,
                                   const float* w_bias, const float* a_bias, const float* v_bias, const float* k_k,
                                   const float* k_a, float* v_first, int layer0, const int32_t* lengths, float* r,
                                   float* w, float* k, float* v, float* a, float* b, float* k_bonus, int64_t B,
                                   int64_t T, int64_t H, void* stream);

/* ───────────────────────────── host-side format work (CPU) ───────────────────────────── */

/* rwkvqUnpack6x8 (Sources/RWKVQuant/RwkvqFile.swift:171-181): n_groups × 6 bytes
 * → n_groups × 8 values in 0..63, LSB-first. */
rwkv_status rwkv_unpack6x8(const uint8_t* in, int64_t n_groups, int32_t* out);

/* rwkvqSb6ToK3 (RwkvqFile.swift:189-212).  Disk buffers: codes_packed
 * [OUT, IN/32·16], qh / qh2 [OUT, IN/32·4] (NULL when absent), gw_qsqm
 * [OUT, IN/256, 12], gw_d / gw_dm [OUT, IN/256] fp16 bits.  Writes the K3
 * qblk / qsqm / ddm described at rwkv_sb6_dequant.  Pure byte permutation. */
rwkv_status rwkv_sb6_to_k3(const uint8_t* codes_packed, const uint8_t* qh, const uint8_t* qh2,
                           const uint8_t* gw_qsqm, const uint16_t* gw_d, const uint16_t* gw_dm,
                           int64_t OUT, int64_t IN, uint8_t* qblk, uint8_t* qsqm, uint16_t* ddm);

/* sym 6-bit interleave (RwkvqFile.swift:437-449): per 32-column pair
 * codes_packed[16] ‖ qh[4] ‖ qh2[4]. */
rwkv_status rwkv_sym_interleave(const uint8_t* codes_packed, const uint8_t* qh, const uint8_t* qh2,
                                int64_t OUT, int64_t IN, uint8_t* qblk);

/* Encoders.  NOT in the reference (its files come from the external
 * rwkv-quant project); min/max per block + 6-bit super-block scales, see
 * swiftrwkv_amd/csrc/host.cpp.  Outputs are the DISK layout above. */
rwkv_status rwkvq_encode_sb6(const float* w, int64_t OUT, int64_t IN, int bits,
                             uint8_t* codes_packed, uint8_t* qh, uint8_t* qh2,
                             uint8_t* gw_qsqm, uint16_t* gw_d, uint16_t* gw_dm, int nthreads);
rwkv_status rwkvq_encode_sym(const float* w, int64_t OUT, int64_t IN, int bits,
                             uint8_t* codes, uint8_t* codes_packed, uint8_t* qh, uint8_t* qh2,
                             uint8_t* gw_qs, uint16_t* gw_d, int nthreads);

/* Read-only memory-mapped safetensors container (RwkvqContainer,
 * RwkvqFile.swift:31-162): rejects torch zip/pickle files, header lengths
 * outside the file, unknown dtypes and data offsets that disagree with
 * shape × dtype. */
typedef struct rwkvq_file rwkvq_file;
rwkv_status rwkvq_open(const char* path, rwkvq_file** out);
void rwkvq_close(rwkvq_file* f);
int64_t rwkvq_count(const rwkvq_file* f);
/* Entry `i` in name order.  dtype is the safetensors name ("U8", "F16" ...). */
rwkv_status rwkvq_entry(const rwkvq_file* f, int64_t i, const char** name, const char** dtype,
                        int* ndim, const int64_t** shape, const void** data, int64_t* nbytes);
/* "__metadata__" string value for `key`, or NULL. */
const char* rwkvq_metadata(const rwkvq_file* f, const char* key);

/* The .rwkvq manifest (the "rwkvq" JSON string of __metadata__), validated as
 * a whole against the container's buffers: replaces the checks of
 * RwkvqSidecar.init(rwkvq:only:fusingSym:) (Sources/RWKVQuant/RwkvqFile.swift:254-492)
 * with the tensor kinds of RwkvqKind / RwkvqTensorInfo (RwkvqSidecar.swift:60-99).
 * Beyond the reference's checks, every buffer an sb6 / sym / asym decode reads
 * must hold exactly the element count its (OUT, IN) needs, so no repack or
 * kernel can read past a buffer of an accepted file. */
typedef enum { RWKVQ_DENSE = 0, RWKVQ_SB6 = 1, RWKVQ_SYM = 2, RWKVQ_ASYM = 3, RWKVQ_RTN = 4 } rwkvq_kind;

/* What a rejected manifest was rejected for (the RwkvqError cases
 * malformedManifest / missingBuffer / shapeMismatch, RwkvqSidecar.swift:25-56). */
typedef enum {
    RWKVQ_FINDING_NONE = 0,
    RWKVQ_FINDING_MALFORMED = 1,
    RWKVQ_FINDING_MISSING_BUFFER = 2,
    RWKVQ_FINDING_SHAPE = 3
} rwkvq_finding_kind;

typedef struct {
    int kind;              /* rwkvq_finding_kind */
    char tensor[192];      /* manifest key ("" for file-level problems) */
    char buffer[32];       /* field name ("gw_qsqm" ...) for MISSING_BUFFER / SHAPE */
    int n_expected, n_got; /* SHAPE: the dims the layout needs / the file holds */
    int64_t expected[4], got[4];
} rwkvq_finding;

typedef struct {
    const char* key;       /* valid while the manifest lives */
    int kind;              /* rwkvq_kind */
    int ndim;
    int64_t shape[8];      /* manifest shape; [OUT, IN] for matrices */
    int bits, xbits;       /* code width; sb6 high-bit planes (0..2) */
    int group_size, super_block;
    int transposed;        /* stored [in, out]: the Linear convention needs a turn */
    int packed;            /* rtn: codes_packed present */
    int64_t outliers;      /* rtn: outlier count */
} rwkvq_tensor;

typedef struct {
    int format_version;
    const char* naming;    /* "world" when absent */
    int64_t n_layer, n_embd, head_size, vocab_size;
} rwkvq_model;

typedef struct rwkvq_manifest rwkvq_manifest;
/* Reads and checks the manifest of `f` (which must stay open while the
 * manifest is used).  On RWKV_E_FORMAT, `finding` (may be NULL) says what was
 * wrong and rwkv_last_error() says it in words. */
rwkv_status rwkvq_manifest_read(const rwkvq_file* f, int max_format_version, rwkvq_manifest** out,
                                rwkvq_finding* finding);
void rwkvq_manifest_free(rwkvq_manifest* m);
int64_t rwkvq_manifest_count(const rwkvq_manifest* m);
/* Entry `i` in key order. */
rwkv_status rwkvq_manifest_tensor(const rwkvq_manifest* m, int64_t i, rwkvq_tensor* out);
rwkv_status rwkvq_manifest_model(const rwkvq_manifest* m, rwkvq_model* out);
/* Entry `i` of an sb6 / sym matrix in the loader layouts (rwkv_sb6_to_k3 /
 * rwkv_sym_interleave of its disk buffers), written to caller host buffers:
 * qblk [OUT, IN/32·(16+4·xbits)], qsqm [OUT, IN/32·2], ddm [OUT, IN/256·2];
 * sym: qblk [OUT, IN] (8-bit) or [OUT, IN/32·24] (6-bit), qs [OUT, IN/16],
 * d [OUT, IN/256].  Rows are packed densely, so pointing into row i·OUT of a
 * larger buffer places a matrix inside a row-concatenated group. */
rwkv_status rwkvq_read_sb6(const rwkvq_file* f, const rwkvq_manifest* m, int64_t i, uint8_t* qblk,
                           uint8_t* qsqm, uint16_t* ddm);
rwkv_status rwkvq_read_sym(const rwkvq_file* f, const rwkvq_manifest* m, int64_t i, uint8_t* qblk,
                           uint8_t* qs, uint16_t* d);

/* ───────────────────────────── measurement ───────────────────────────── */

/* Measurement hook, no counterpart in the reference (its benches time whole
 * MLX evals).  Arms the NEXT kernel launch made by this library on the
 * calling thread to record its own start / stop timestamps into the given
 * hipEvent_t pair (hipExtLaunchKernelGGL), so elapsed time between them is
 * the kernel alone.  NULL, NULL disarms. */
rwkv_status rwkv_time_next_launch(void* start_event, void* stop_event);

/* ───────────────────────────── counters ───────────────────────────── */

typedef struct {
    int64_t seq_fwd;        /* wkv7SequenceLaunches (WKV7.swift:181) */
    int64_t chunk_fwd;
    int64_t train_fwd;      /* wkv7TrainForwardLaunches (WKV7Train.swift:358) */
    int64_t train_bwd;
    int64_t step;           /* stepKernelCalls (X070Backbone.swift) */
    int64_t tail;
    int64_t sb6_dequant;
    int64_t sym_dequant;
    int64_t sb6_gemv;       /* rwkvqSb6GEMVCalls */
    int64_t sym_gemv;       /* rwkvqSymGEMVCalls */
    int64_t sym_fused;      /* rwkvqSymFusedCalls */
    int64_t step_tail;      /* rwkv_wkv7_step_tail launches (no reference counter) */
    int64_t sb6_fused;      /* rwkv_sb6_gemv_fused launches (no reference counter) */
    int64_t sym_rows;       /* rwkv_sym_rows launches (no reference counter) */
    int64_t x070;           /* layer_norm / x070_* launches (no reference counter) */
    int64_t sb6_gemm;       /* rwkv_sb6_gemm launches (no reference counter) */
    int64_t seq_chunked;    /* rwkv_wkv7_seq_fwd_chunked launches (no reference counter) */
    int64_t sb6_batch;      /* rwkv_sb6_gemv_batch calls (no reference counter) */
    int64_t sym_gemm;       /* rwkv_sym_gemm launches (no reference counter) */
} rwkv_counters;

void rwkv_get_counters(rwkv_counters* out);
void rwkv_reset_counters(void);

#ifdef __cplusplus
}
#endif

#endif /* RWKV_HIP_H */
