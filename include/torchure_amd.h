/*
 * torchure_amd.h -- C ABI of the MI355X (gfx950) mixed-precision optimizer step.
 *
 * The library replaces the device work of torchure's optimizer tail
 * (torchure/train/trainer.py:391-397):
 *   clip_grad_norm  (torchure/core/grad_helper.py:8-34)
 *       = torch._foreach_norm + stack + vector_norm + clamp + torch._foreach_mul_
 *   optimizer.step() (torch.optim.AdamW(fused=True), built at torchure/optimizer/builder.py:46)
 *       = torch._foreach_add_(state_steps, 1) + torch._fused_adamw_
 *         (torch/optim/adam.py:877-895; device math in
 *          torch/include/ATen/native/hip/fused_adam_utils.cuh:22-199,
 *          launcher signature torch/include/ATen/native/hip/fused_adam_impl.cuh:8-21)
 *   plus the bf16 working-copy refresh that autocast performs at every forward
 *   (torchure/train/trainer.py:374; rounding rule torch/headeronly/util/BFloat16.h:100-114).
 *
 * Conventions
 *   - Every pointer named d_* is device memory; h_* is host memory.
 *   - Nothing here allocates device memory or synchronises the stream: all work is
 *     enqueued on `stream` (a hipStream_t passed as void*; NULL = the null stream).
 *   - Return value: TM_OK (0) or a negative TM_E* code; tm_last_error() gives a
 *     thread-local message for the last failure.
 *   - Tensors are described by tm_tensor_t records in device memory and split into
 *     fixed-size chunks by a tm_chunk_t table (device memory) built with
 *     tm_fill_chunks(). Both tables are plain data owned by the caller.
 */
#ifndef TORCHURE_AMD_H
#define TORCHURE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TM_ABI_VERSION 3

/* status codes */
#define TM_OK 0
#define TM_EINVAL (-1)   /* bad argument (null pointer, size out of range) */
#define TM_ELAUNCH (-2)  /* kernel launch failed */

/* tm_tensor_t.flags */
#define TM_GRAD_BF16 0u  /* grad is bfloat16 (uint16 storage) */
#define TM_GRAD_F32 1u   /* grad is float32 (e.g. an fp32 accumulation buffer) */
#define TM_FLAG_CLIP 2u  /* multiply the grad by *d_coef before use (deferred clip) */

/* Largest number of hyper-parameter groups one call accepts. */
#define TM_MAX_GROUPS 16

/* Chunk granularity: chunk_elems must be a positive multiple of this. */
#define TM_CHUNK_ALIGN 2048

/* Number of partial sums the grad-norm pass writes (fixed, so the reduction
 * order -- and therefore the result bits -- never depend on the device). */
#define TM_NORM_PARTIALS 2048

/*
 * One tensor of the parameter list (64 bytes, device memory).
 *   master      fp32 master weights, updated in place (torch: the nn.Parameter)
 *   exp_avg     fp32 first moment, updated in place   (state['exp_avg'])
 *   exp_avg_sq  fp32 second moment, updated in place  (state['exp_avg_sq'])
 *   grad        bf16 or fp32 gradient (flags), read only
 *   param_bf16  bf16 working copy written as RNE(master) after the update, or 0
 *   step        fp32 0-d step counter, incremented in place (state['step'])
 *   numel       element count (0 allowed: the step still advances)
 *   group       index into the tm_hyper_t array of the call
 *   flags       TM_GRAD_* | TM_FLAG_CLIP
 * The norm / scale / accumulate entry points read only grad, numel and flags.
 * Preconditions (the records live in device memory, so the library cannot check them
 * without a synchronisation): step is non-null; master, exp_avg, exp_avg_sq and grad are
 * non-null when numel > 0 and hold numel elements; tensors do not overlap. A record whose
 * group is outside [0, n_groups) is not stepped with another group's hyper-parameters: the
 * step poisons it instead (its step counter, master, moments and bf16 copy become NaN).
 */
typedef struct tm_tensor {
  uint64_t master;
  uint64_t exp_avg;
  uint64_t exp_avg_sq;
  uint64_t grad;
  uint64_t param_bf16;
  uint64_t step;
  int64_t numel;
  int32_t group;
  uint32_t flags;
} tm_tensor_t;

/* One work item: chunk `chunk` of tensor `tensor`. For the norm, scale, cast and accumulate
 * entry points it covers elements [chunk*chunk_elems, min((chunk+1)*chunk_elems, numel)),
 * so a table may list any subset of a tensor's chunks. tm_adamw_step and
 * tm_adamw_step_noalloc are different: their table must list every chunk of each tensor,
 * 0 .. ceil(numel/chunk_elems)-1, exactly once, as tm_fill_chunks writes it. The update lays
 * a tensor's slices on 1 KiB boundaries of its arrays, so the elements one of its chunks
 * covers are shifted by up to 255 and chunk 0 also takes the tensor's last elements; that
 * mapping is internal to the kernel, and only the whole set of a tensor's chunks is
 * guaranteed to cover each element once.
 * A call takes at most 4,294,967,295 chunks (32-bit indices); larger
 * tables return TM_EINVAL. The streaming kernels cover a chunk with chunk_elems / 256
 * one-wave workgroups and split a table over as many launches as the 2^32 work-item
 * limit of a launch requires. */
typedef struct tm_chunk {
  uint32_t tensor;
  uint32_t chunk;
} tm_chunk_t;

/* tm_accum_t.flags */
#define TM_ACCUM_ASSIGN 1  /* acc = (float)micro, acc is not read (first micro-step) */

/* One tensor of a micro-step accumulation list (32 bytes, device memory):
 * acc (fp32, updated in place) += micro (bf16), numel elements; with TM_ACCUM_ASSIGN
 * acc = micro instead, as autograd assigns the first grad (torch's AccumulateGrad
 * stores the first incoming grad and adds later ones). micro may be 0: the
 * accumulator is then left as is and only enters the norm. */
typedef struct tm_accum {
  uint64_t acc;
  uint64_t micro;
  int64_t numel;
  int64_t flags;
} tm_accum_t;

/* Hyper-parameters of one param group, as torch.optim.AdamW holds them
 * (python floats = double): torch/optim/adam.py:35-113, fused_adam_utils.cuh:110-121. */
typedef struct tm_hyper {
  double lr;
  double beta1;
  double beta2;
  double weight_decay;
  double eps;
} tm_hyper_t;

/* ---- library / table helpers (host only, no GPU work) ---- */

int tm_abi_version(void);
const char* tm_last_error(void);

/* Device workspace bytes needed by tm_grad_norm / tm_adamw_step for n_tensors. */
size_t tm_workspace_bytes(int64_t n_tensors);

/* Number of chunks the tensors split into (zero-size tensors give none). */
int64_t tm_count_chunks(const int64_t* h_numels, int64_t n_tensors, int64_t chunk_elems);

/* Writes the chunk table into h_out (capacity `cap` entries) in tensor order.
 * Returns the number written, or a negative TM_E* code. */
int64_t tm_fill_chunks(const int64_t* h_numels, int64_t n_tensors, int64_t chunk_elems,
                       tm_chunk_t* h_out, int64_t cap);

/* ---- device entry points ---- */

/*
 * Global L2 norm of all grads, deterministic two-pass (no atomics).
 * Replaces torch._foreach_norm + torch.stack + torch.linalg.vector_norm
 * (torchure/core/grad_helper.py:17-18) and the clip coefficient
 * clamp(max_norm / (total + 1e-6), max=1.0) (grad_helper.py:32, evaluated as
 * reciprocal-then-multiply per torch/_tensor.py:1119-1122).
 *   d_norm  receives the pre-clip norm (fp32, grad_helper.py:34)
 *   d_coef  receives the clip coefficient when clip != 0 (else untouched; may be NULL)
 *   d_ws    at least tm_workspace_bytes(n_tensors) bytes
 */
int tm_grad_norm(const tm_tensor_t* d_tensors, int64_t n_tensors, const tm_chunk_t* d_chunks,
                 int64_t n_chunks, int64_t chunk_elems, float max_norm, int clip, void* d_ws,
                 float* d_norm, float* d_coef, void* stream);

/*
 * In-place grad *= *d_coef for every tensor (the eager clip).
 * Replaces torch._foreach_mul_(grads, clip_coef) (grad_helper.py:33): fp32 grads
 * get one fp32 multiply; bf16 grads are widened and multiplied by the coefficient
 * rounded to bf16 (torch holds the scalar in the list's dtype), then rounded back RNE.
 */
int tm_grad_scale(const tm_tensor_t* d_tensors, int64_t n_tensors, const tm_chunk_t* d_chunks,
                  int64_t n_chunks, int64_t chunk_elems, const float* d_coef, void* stream);

/*
 * One fused AdamW step over every tensor in the table, all groups in one launch.
 * Replaces torch._foreach_add_(state_steps, 1) + torch._fused_adamw_
 * (torch/optim/adam.py:877-895; math fused_adam_utils.cuh:22-92,106-199), fuses
 * the deferred clip scale (tensors with TM_FLAG_CLIP read *d_coef) and the bf16
 * working-copy refresh (param_bf16 != 0).
 *   h_groups  n_groups (1..TM_MAX_GROUPS) host records; tm_tensor_t.group indexes them
 *   d_chunks  every chunk of every tensor exactly once (tm_fill_chunks), see tm_chunk_t
 *   d_coef    clip coefficient (device fp32) applied to TM_FLAG_CLIP tensors; NULL means
 *             no tensor is scaled (TM_FLAG_CLIP is then ignored)
 *   d_ws      at least tm_workspace_bytes(n_tensors) bytes
 */
int tm_adamw_step(const tm_tensor_t* d_tensors, int64_t n_tensors, const tm_chunk_t* d_chunks,
                  int64_t n_chunks, int64_t chunk_elems, const tm_hyper_t* h_groups,
                  int32_t n_groups, const float* d_coef, void* d_ws, void* stream);

/* Largest n_tensors tm_adamw_step_noalloc accepts (the entries of its static scratch). */
#define TM_NOALLOC_MAX_TENSORS 16384

/*
 * tm_adamw_step without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It has
 * no counterpart in the reference. Its per-tensor constants live in a static device array of
 * TM_NOALLOC_MAX_TENSORS entries (1 MiB on every GPU the library runs on, held until the
 * process ends); a call with more tensors returns TM_EINVAL. It calls no allocating routine.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams,
 * or two host threads) race and must be serialised by the caller. Results equal
 * tm_adamw_step's, bit for bit. The chunk table follows tm_adamw_step's rule (every chunk of
 * every tensor exactly once). The hyper-parameters (h_groups: lr, betas, weight decay, eps)
 * are copied into the launch's kernel arguments at call time: a captured HIP graph replays
 * the lr it was captured with, so a schedule (WSD or any other) needs the graph captured
 * again, or its prep kernel node's parameters updated, whenever lr changes.
 */
int tm_adamw_step_noalloc(const tm_tensor_t* d_tensors, int64_t n_tensors, const tm_chunk_t* d_chunks,
                          int64_t n_chunks, int64_t chunk_elems, const tm_hyper_t* h_groups,
                          int32_t n_groups, const float* d_coef, void* stream);

/*
 * Micro-step gradient accumulation: d_acc[i] (fp32) += (float)d_micro[i] (bf16),
 * over `numel` elements. The fp32 accumulation buffer is what torch autograd
 * builds in p.grad across micro-batches (torchure/train/trainer.py:383-390).
 */
int tm_grad_accumulate_bf16(float* d_acc, const uint16_t* d_micro, int64_t numel, void* stream);

/*
 * Micro-step accumulation over a list of tensors, one launch: acc += micro for every
 * entry (the fp32 .grad accumulation of torchure/train/trainer.py:383-390).
 * With with_norm != 0 (the last micro-step) the same pass also produces the global
 * L2 norm of the accumulated grads into d_norm, bit-identical to tm_grad_norm on the
 * resulting fp32 buffers with the same chunk table -- the separate norm read pass of
 * torch._foreach_norm (torchure/core/grad_helper.py:17-18) disappears. The pass writes
 * one fp64 partial per 256-element slice into the workspace, which two small launches
 * then reduce in a fixed order.
 *   d_ws, ws_bytes  with_norm != 0: at least tm_accum_norm_workspace_bytes(n_chunks,
 *                   chunk_elems) bytes (else unused; may be NULL)
 * (ABI version 2 added ws_bytes; version 1 took a 16 KB workspace.)
 */
size_t tm_accum_norm_workspace_bytes(int64_t n_chunks, int64_t chunk_elems);
int tm_grad_accumulate_list(const tm_accum_t* d_list, int64_t n_list, const tm_chunk_t* d_chunks,
                            int64_t n_chunks, int64_t chunk_elems, int with_norm, void* d_ws, size_t ws_bytes,
                            float* d_norm, void* stream);

/* Clip coefficient from a norm already on the device:
 * clamp(max_norm / (norm + 1e-6), max=1.0) as in tm_grad_norm (grad_helper.py:32). */
int tm_clip_coef(const float* d_norm, float max_norm, float* d_coef, void* stream);

/* Writes RNE(src) into dst (bf16 working-copy refresh without an update).
 * Rounding rule of torch/headeronly/util/BFloat16.h:100-114 (NaN -> 0x7FC0). */
int tm_cast_bf16(uint16_t* d_dst, const float* d_src, int64_t numel, void* stream);

/*
 * The same cast over a list, one launch: param_bf16 = RNE(master) for every record whose
 * param_bf16 is non-zero (only master, param_bf16 and numel are read). Replaces the per-weight
 * cast autocast performs at every forward (torchure/train/trainer.py:374) for the whole list;
 * used to create and to refresh the bf16 working copies.
 */
int tm_cast_bf16_list(const tm_tensor_t* d_tensors, int64_t n_tensors, const tm_chunk_t* d_chunks,
                      int64_t n_chunks, int64_t chunk_elems, void* stream);

/*
 * dst = src over nbytes (a multiple of 16; both pointers 16-byte aligned; the ranges must not
 * overlap), one wave per KiB with non-temporal 16-byte accesses. No counterpart in the
 * reference: it is the best 1:1 read/write stream this library's launch shapes reach on
 * MI355X, which bench.py times beside the update as the device's measured streaming ceiling.
 */
int tm_stream_copy(void* d_dst, const void* d_src, int64_t nbytes, void* stream);

/* ---- chunked fused linear + cross-entropy (torchure/loss/fused_linear_ce.py) ---- */

/*
 * One fused pass over a chunk of bf16 logits (rows x vocab, row stride ld elements),
 * replacing the per-chunk softmax math of torchure/loss/fused_linear_ce.py:40-52:
 *   lse = logsumexp(float(logits)), row_loss = lse - logits[label] (0 on ignored rows),
 *   logits <- bf16(exp(logits - lse) - onehot(label)) on valid rows, 0 on ignored rows.
 * Labels are int64; a row is ignored when label == ignore_index. A label outside [0, vocab)
 * that is not ignore_index gives that row a NaN loss (the reference fails on it in gather).
 */
int tm_ce_rows_bf16(uint16_t* d_logits, int64_t ld, const int64_t* d_labels, int64_t rows,
                    int64_t vocab, int64_t ignore_index, float* d_row_loss, void* stream);

/*
 * The row losses of tm_ce_rows_bf16 without the gradient: the logits are only read. Same
 * arithmetic, so the same bits. For a call whose inputs need no gradient (evaluation under
 * torch.no_grad), where the reference's forward (fused_linear_ce.py:63-93) still computes
 * and discards the gradients.
 */
int tm_ce_rows_loss_bf16(const uint16_t* d_logits, int64_t ld, const int64_t* d_labels, int64_t rows,
                         int64_t vocab, int64_t ignore_index, float* d_row_loss, void* stream);

/*
 * The same chunk math on fp32 logits, for fp32 hidden states outside autocast: there the
 * reference's products are fp32 GEMMs (fused_linear_ce.py:38,52,57, w = weight.to(fp32) at :65)
 * and its softmax runs on fp32 logits (:39-51). lse = logsumexp(logits), row_loss = lse -
 * logits[label] (0 on ignored rows, NaN for a label outside [0, vocab)), and
 * logits <- exp(logits - lse) - onehot(label) in fp32 (0 on ignored rows): the fp32 difference,
 * then a full-precision exp, as the reference's exp(logits - lse). tm_ce_rows_loss_f32 gives
 * the same row losses and only reads the logits.
 */
int tm_ce_rows_f32(float* d_logits, int64_t ld, const int64_t* d_labels, int64_t rows, int64_t vocab,
                   int64_t ignore_index, float* d_row_loss, void* stream);
int tm_ce_rows_loss_f32(const float* d_logits, int64_t ld, const int64_t* d_labels, int64_t rows,
                        int64_t vocab, int64_t ignore_index, float* d_row_loss, void* stream);

/*
 * Deterministic loss reduction (fused_linear_ce.py:76-90): d_out3[0] = sum of row
 * losses, d_out3[1] = n_valid = max(1, count(label != ignore_index)),
 * d_out3[2] = d_out3[0] / d_out3[1] (the mean loss).
 */
int tm_ce_loss(const float* d_row_loss, const int64_t* d_labels, int64_t rows, int64_t ignore_index,
               float* d_out3, void* stream);

/*
 * Backward scaling in place (fused_linear_ce.py:117-126): scale = *d_grad_out / *d_n_valid;
 * grad_h (bf16) *= bf16(scale), grad_w (fp32, may be NULL with nw = 0) *= scale.
 */
int tm_ce_scale_grads(uint16_t* d_grad_h, int64_t nh, float* d_grad_w, int64_t nw,
                      const float* d_grad_out, const float* d_n_valid, void* stream);

/*
 * grad_W hand-over of one chunk (fused_linear_ce.py:80-81 `grad_weight += gw`, and for the
 * last chunk also :126 `grad_weight.mul_(scale)`):
 *   d_grad_w[i] = ((accumulate ? d_grad_w[i] : +0.0f) + float(d_chunk[i])) [* scale]
 * with scale = *d_grad_out / *d_n_valid when d_grad_out is given (both or neither).
 * accumulate = 0 replaces the zero fill + first `+=` (no read of d_grad_w); the
 * scaled form lets the last chunk's bf16 grad_W wait for backward and be folded in
 * together with the scaling, one pass instead of two.
 */
int tm_ce_grad_w(float* d_grad_w, const uint16_t* d_chunk, int64_t nw, int accumulate,
                 const float* d_grad_out, const float* d_n_valid, void* stream);

/*
 * The same hand-over for two consecutive chunks in one pass (fused_linear_ce.py:80-81 run
 * for chunk k and then chunk k+1, and :126 when d_grad_out is given):
 *   d_grad_w[i] = (((accumulate ? d_grad_w[i] : +0.0f) + float(d_chunk[i])) + float(d_chunk2[i])) [* scale]
 * the reference's fp32 additions in its order, reading and writing the accumulator once
 * for both chunks.
 */
int tm_ce_grad_w2(float* d_grad_w, const uint16_t* d_chunk, const uint16_t* d_chunk2, int64_t nw,
                  int accumulate, const float* d_grad_out, const float* d_n_valid, void* stream);

/*
 * The same hand-over for n_chunks (1 to 8) consecutive chunks in one pass
 * (fused_linear_ce.py:80-81 run for each of them in order, and :126 when d_grad_out is given):
 *   d_grad_w[i] = (((accumulate ? d_grad_w[i] : +0.0f) + float(c0[i])) + float(c1[i]) + ...) [* scale]
 * h_chunks is a host array of n_chunks device pointers (bf16, nw elements each), read at the
 * call. The reference's fp32 additions in its order: the bits of one `+=` per chunk, for one
 * read and one write of the fp32 accumulator per n_chunks chunks.
 */
int tm_ce_grad_w_fold(float* d_grad_w, const uint16_t* const* h_chunks, int n_chunks, int64_t nw, int accumulate,
                      const float* d_grad_out, const float* d_n_valid, void* stream);

/*
 * grad_hidden of fp32 hidden states (fused_linear_ce.py:68,80,120 under autocast: the
 * buffer has the hidden states' dtype, holds the widened bf16 GEMM result and is scaled
 * in place in fp32): d_dst[i] = float(d_src[i]) * (*d_grad_out / *d_n_valid), -0 kept.
 */
int tm_ce_widen_scale(float* d_dst, const uint16_t* d_src, int64_t n, const float* d_grad_out,
                      const float* d_n_valid, void* stream);

/*
 * grad_hidden of one chunk, fused_linear_ce.py:52 `grad_hidden = grad_logits @ weight` (and its
 * store at :79), for the chunk shapes where a split-K GEMM pays: rows and dim positive
 * multiples of 256, vocab a multiple of 64, all pointers 16-byte aligned, every matrix
 * contiguous. d_grad_h (rows x dim) = bf16(d_grad_logits (rows x vocab) @ d_w) with fp32
 * accumulation, d_w the weight as the op holds it (vocab x dim, row-major). The K range
 * is split into S ranges whose fp32 partial tiles go to d_ws and are summed in the fixed order
 * 0..S-1 before the single bf16 rounding: the result is deterministic; it differs from another
 * GEMM's only by fp32 summation order. d_ws holds tm_ce_grad_h_workspace_bytes(rows, vocab, dim)
 * bytes (S x rows x dim fp32, 0 for shapes the GEMM does not take); calls that share a
 * workspace on one stream are ordered, on different streams they race. (ABI version 3: d_w is
 * the weight itself; version 2 took its transpose, made by a tm_ce_transpose_bf16 since removed.)
 */
size_t tm_ce_grad_h_workspace_bytes(int64_t rows, int64_t vocab, int64_t dim);
int tm_ce_grad_h_bf16(uint16_t* d_grad_h, const uint16_t* d_grad_logits, const uint16_t* d_w, int64_t rows,
                      int64_t vocab, int64_t dim, void* d_ws, size_t ws_bytes, void* stream);

/*
 * The logits of one chunk, fused_linear_ce.py:38 `logits = h @ w.t()` (a bf16 matmul: fp32
 * accumulation, bf16 result): d_logits (rows x vocab) = bf16(d_hidden (rows x dim) @ d_weight^T)
 * with d_weight the vocab x dim head, all three contiguous and 16-byte aligned, dim a positive
 * multiple of 64 (rows and vocab any positive sizes). RNE rounding of the fp32 sum over dim;
 * deterministic. Replaces the library GEMM torch.matmul dispatches there.
 */
int tm_ce_logits_bf16(uint16_t* d_logits, const uint16_t* d_hidden, const uint16_t* d_weight, int64_t rows,
                      int64_t vocab, int64_t dim, void* stream);

/*
 * The weight gradient of one chunk, fused_linear_ce.py:57 `gw = grad_logits.t() @ h` (a bf16
 * matmul: fp32 accumulation, bf16 result): d_grad_w (vocab x dim) = bf16(d_grad_logits^T @
 * d_hidden) with d_grad_logits rows x vocab and d_hidden rows x dim, all contiguous and 16-byte
 * aligned, rows a positive multiple of 64, vocab and dim positive multiples of 8. RNE rounding
 * of the fp32 sum over rows; deterministic. Replaces the library GEMM torch.matmul dispatches
 * there; the fp32 accumulation of the chunks stays tm_ce_grad_w_fold's.
 */
int tm_ce_grad_w_bf16(uint16_t* d_grad_w, const uint16_t* d_grad_logits, const uint16_t* d_hidden, int64_t rows,
                      int64_t vocab, int64_t dim, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TORCHURE_AMD_H */
