/*
 * weightferry.h -- C ABI of the MI355X (gfx950) quantized-weight hot path.
 *
 * One shared library, libweightferry_hip.so, built from comfyui-weightferry_amd/csrc/. Plain pointers and sizes
 * only; every device pointer is memory the caller allocated (the library never allocates or frees device memory
 * on these paths). `stream` is a hipStream_t (NULL = the default stream); every call is asynchronous on it and
 * never synchronises the host.
 *
 * Return codes: WF_OK (0) on success; WF_EUNSUPPORTED (-2) when the call is "not my case" (the reference's
 * Python returns None there and the host application's own code runs); WF_EINVAL (-1) for malformed arguments;
 * WF_EHIP (-3) when a HIP runtime call failed. wf_last_error() gives a thread-local message for the last failure
 * on the calling thread.
 *
 * Dtype codes follow enhancers/gguf_dequant.py:58 of the reference: 0 float16, 1 bfloat16, 2 float32.
 * GGML type ids follow enhancers/gguf_dequant.py:52-56: 2 Q4_0, 3 Q4_1, 6 Q5_0, 7 Q5_1, 8 Q8_0, 10 Q2_K, 11 Q3_K,
 * 12 Q4_K, 13 Q5_K, 14 Q6_K.
 */
#ifndef WEIGHTFERRY_H
#define WEIGHTFERRY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WF_OK 0
#define WF_EINVAL (-1)
#define WF_EUNSUPPORTED (-2)
#define WF_EHIP (-3)

#define WF_F16 0
#define WF_BF16 1
#define WF_F32 2

/* ABI version (bumped on any signature change) and the last error message of the calling thread. */
int wf_abi_version(void);
const char* wf_last_error(void);

/* ---------------------------------------------------------------------------------------------- dequantisation
 * Replaces the Triton launches of `dequantize` / `_dequantize_k` (enhancers/gguf_dequant.py:277-326; kernels
 * `_deq` :136-167 and `_deq_k` :188-256). `src` holds src_bytes of GGUF blocks of type `qtype`; `out` receives
 * n_values values of dtype out_dt, each computed with the reference's rounding chain in the dequant dtype mid_dt.
 * WF_EUNSUPPORTED when qtype / dtypes are not handled or src_bytes does not hold exactly n_values values (the
 * reference returns None there, :280-286,312-320), or when src / out are not 16-byte aligned. */
int wf_dequant(const void* src, int64_t src_bytes, int qtype, int mid_dt, int out_dt, void* out, int64_t n_values,
               void* stream);

/* LoRA add on a GGUF weight: replaces the Triton kernel `_deq_add` (enhancers/gguf_dequant.py:99-133) as
 * `_add_loras` launches it once per LoRA (:387-409). out[i] = OUT(w + OUT(diff[i] * scale)) for i < n_values, the
 * product, the sum and each rounding on their own; w is the dequantisation of `src` exactly as wf_dequant gives it
 * (the first LoRA, DEQ on) when src is not NULL, else the value already in out (a later LoRA; qtype, src_bytes
 * and mid_dt are then ignored). diff: float32 [n_values], comfy's up @ down of one LoRA; scale = strength *
 * alpha / rank. The reference dequantises a K-quant by its own kernel and adds every LoRA afterwards; here the
 * first add is fused into the K-quant dequantisation too (the same values). out and diff 16-byte aligned. */
int wf_dequant_add(const void* src, int64_t src_bytes, int qtype, int mid_dt, int out_dt, const float* diff,
                   float scale, void* out, int64_t n_values, void* stream);

/* ---------------------------------------------------------------------------------------------- int8 W8A8 path
 * Per-row int8 quantisation of bf16 activations: replaces the Triton `_quant_row` with PRE_NONE
 * (enhancers/fused_kernels.py:137-174, launched at enhancers/fused_int8.py:172-176) and kitchen's
 * quantize_int8_rowwise_convrot64 (enhancers/fused_int8.py:178-181). mode 0: plain per-token (K % 16 == 0,
 * K <= 32768); mode 1: ConvRot 256-groups (K % 256 == 0, K <= 32768). x: bf16 [M, K] row-major; xq: int8 [M, K];
 * xs: float32 [M]. x and xq 16-byte aligned. */
int wf_quant_rows_i8(const void* x_bf16, int64_t M, int64_t K, int mode, int8_t* xq, float* xs, void* stream);

/* The ConvRot quantisation (mode 1 above) with an operation applied to each value first: replaces the Triton
 * `_quant_row` with PRE 1..3 (enhancers/fused_kernels.py:137-163) as `_quantise_pre` launches it for a pending input
 * (enhancers/fused_int8.py:60-75). pre 0: none; 1 GELU: y = table[bits(x)], s_bf16 = torch's GELU of all 65536 bf16
 * values (:94-105); 2 MOD: y = bf16(bf16(x * s1) + shift) with s_bf16 = s1 = 1 + scale and shift_bf16 = shift, both
 * bf16 [M / rows_per_group, K], row r using group r / rows_per_group (:28-39); 3 LNMOD: LayerNorm without affine
 * first -- mean and variance by the reference's Welford order (:84-136), rstd = 1 / sqrt(var + eps) correctly rounded
 * where the reference uses the NVIDIA approximation rsqrt.approx.f32 -- rounded to bf16, then MOD. K % 256 == 0,
 * K <= 32768 (LNMOD: K % 512 == 0); s / shift 16-byte aligned for MOD / LNMOD. */
int wf_quant_rows_i8_pre(const void* x_bf16, int64_t M, int64_t K, int pre, const void* s_bf16, const void* shift_bf16,
                         int64_t rows_per_group, float eps, int8_t* xq, float* xs, void* stream);

/* out[m, n] = OUT((float(acc[m, n]) * xs[m]) * ws[n] (+ bias[n])), acc = sum_k xq[m, k] * wq[n, k] exactly in
 * int32: replaces kitchen's cutlass_int8_dequant (enhancers/fused_int8.py:191-206; the reference returns None and
 * falls back where this returns WF_EUNSUPPORTED). wq is [N, K] (row = output channel); bias (nullable) has dtype
 * out_dt; out_dt is WF_BF16 or WF_F16. K % 16 == 0, xq / wq 16-byte aligned. */
int wf_linear_i8(const int8_t* xq, const int8_t* wq, const float* xs, const float* ws, const void* bias, void* out,
                 int out_dt, int64_t M, int64_t N, int64_t K, void* stream);

/* out = bf16(resid + gate[m / rows_per_group] * bf16((float(acc) * xs[m]) * ws[n])): wf_linear_i8's bf16 output
 * followed by torch.addcmul(resid, gate, out) on bf16 tensors (the product exact in float32, the sum rounded once
 * to float32, then to bf16) -- replaces kitchen's cutlass_int8_dequant_residual, which the reference states gives
 * those bits (enhancers/fused_int8.py:212-268: x_res + gate * linear(x) per (batch, frame) group of rows;
 * enhancers/fused_block.py:24-26). gate: bf16 [M / rows_per_group, N]; resid, out: bf16 [M, N]. */
int wf_linear_i8_residual(const int8_t* xq, const int8_t* wq, const float* xs, const float* ws, const void* gate_bf16,
                          const void* resid_bf16, void* out_bf16, int64_t M, int64_t N, int64_t K,
                          int64_t rows_per_group, void* stream);

/* ------------------------------------------------------------------------------- fused dequant + bf16 GEMM
 * y[m, n] = bf16(sum_k x[m, k] * W[n, k] (+ bias[n])) with W given as GGUF K-quant blocks (qtype 12 Q4_K, 13 Q5_K, 14
 * Q6_K; [N, K] row-major in 256-value super-blocks, wq_bytes = N * K / 256 * block bytes; also qtype 8 Q8_0, 34 bytes
 * per 32 values, at 1-512 rows only, WF_EUNSUPPORTED elsewhere; its panels take 64 rows, and wf_linear_gguf_ws and
 * wf_linear_gguf_noalloc give it the panel form at the K-quants' rows) and dequantised inside the kernel exactly as
 * wf_dequant does with dequant dtype mid_dt and output bf16; float32 accumulation. No reference function does this in
 * one step: it replaces `dequantize` (enhancers/gguf_dequant.py:296-326) followed by ComfyUI-GGUF's
 * torch.nn.functional.linear on the bf16 weight. x: bf16 [M, K], 16-byte aligned; bias: bf16 [N] or NULL; out: bf16
 * [M, N]. K % 256 == 0, K <= 1048576. M <= 64 runs the few-rows forms (the weight streamed once; at 1-3 rows of N <
 * 8192, Q6_K and Q8_0 1-4 rows of N < 16384: workgroups of whole 4-row quads), 65-512 rows the panel form, larger M
 * the tiled form (256 x 320 tiles; Q6_K from 1024 rows 512 x 160). */
int wf_linear_gguf(const void* x_bf16, int64_t M, int64_t K, const void* wq, int64_t wq_bytes, int qtype, int64_t N,
                   const void* bias_bf16, void* out_bf16, int mid_dt, void* stream);

/* wf_linear_gguf with a caller-provided workspace, for the same reference call site (enhancers/gguf_dequant.py:
 * 296-326 followed by ComfyUI-GGUF's F.linear). A narrow, deep product (N <= 2048, K >= 8192, K >= 2 N) with 1 <= M <=
 * 8 rows is split along K over many more workgroups than weight rows allow: each writes float32 partial sums into the
 * workspace, and the last workgroup of each column tile adds them in a fixed order (the result is the same on every
 * run). Workspace: 256-byte aligned, at least the bytes wf_linear_gguf_workspace gives; its first 16 KiB are counters
 * that must be zero on entry and are zero again when the call has run, whatever its shape (a workspace cleared once
 * can be reused by later calls of any shape on the same stream; calls that overlap on one workspace race). With 33-512
 * rows, and with 17-32 rows of a deep product (K >= 2 N), the panel form splits K into slices (at least two
 * super-blocks each), enough to give the chip 256 workgroups: each slice writes float32 partial sums into the
 * workspace past the split form's 16 KiB of counters, which it leaves untouched (16 KiB + S * M * N * 4 bytes), and a
 * second kernel adds them in slice order; up to 64 rows only when K gives more than one slice.
 * wf_linear_gguf_workspace does not know the format and gives the largest need over them. Any other shape does not use
 * the workspace (workspace may be NULL) and is wf_linear_gguf. */
int wf_linear_gguf_workspace(int64_t M, int64_t N, int64_t K, int64_t* bytes);
int wf_linear_gguf_ws(const void* x_bf16, int64_t M, int64_t K, const void* wq, int64_t wq_bytes, int qtype, int64_t N,
                      const void* bias_bf16, void* out_bf16, int mid_dt, void* workspace, int64_t workspace_bytes,
                      void* stream);

/* wf_linear_gguf_ws without the workspace argument: allocates nothing. No counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). The split form's counters and partial sums live in a 16 MiB array the library holds on each GPU
 * it runs on until the process ends; the counters are cleared by a small kernel on `stream` at the start of each call
 * (no memset). A shape that needs more than 16 MiB there returns WF_EUNSUPPORTED with a message. The panel form
 * (the rows of wf_linear_gguf_ws) takes as many K slices as fit the array past the counters (one, and no scratch, at
 * worst; up to 64
 * rows one slice leaves the call to the few-rows kernel). Every call on a GPU shares
 * that GPU's array: calls that overlap on one GPU (on different streams or threads) race. */
int wf_linear_gguf_noalloc(const void* x_bf16, int64_t M, int64_t K, const void* wq, int64_t wq_bytes, int qtype,
                           int64_t N, const void* bias_bf16, void* out_bf16, int mid_dt, void* stream);

/* y[m, n] = bf16(sum_k x[m, k] * w[n, k] (+ bias[n])), float32 accumulation: the GEMM of the two-step flow, after
 * wf_dequant -- replaces ComfyUI-GGUF's torch.nn.functional.linear on the weight that `dequantize`
 * (enhancers/gguf_dequant.py:296-326) returns. x: bf16 [M, K], w: bf16 [N, K], both 16-byte aligned; bias: bf16 [N]
 * or NULL; out: bf16 [M, N]. K % 64 == 0 and M * K, N * K < 2^30, else WF_EUNSUPPORTED (the caller's own GEMM runs).
 * Tiles of 256 x 320, 256 x 256, 256 x 128 or 128 x 160 outputs, whichever fills the chip best. */
int wf_linear_bf16(const void* x_bf16, const void* w_bf16, const void* bias_bf16, void* out_bf16, int64_t M, int64_t N,
                   int64_t K, void* stream);

/* ---------------------------------------------------------------------------------------- block streaming
 * Exact-size page-locked host memory: replaces PinnedHost's cudaHostRegister / cudaHostUnregister
 * (core/tiers/pinned.py:84-129); allocated page-locked (hipHostMalloc) instead of registered after the fact. */
int wf_host_alloc(size_t nbytes, void** ptr);
int wf_host_free(void* ptr);

/* Asynchronous host -> device copy on `stream`: replaces slot_flats[slot].copy_(host_flat, non_blocking=True)
 * (streaming/state.py:142-143). */
int wf_h2d_async(void* dst, const void* src, size_t nbytes, void* stream);

/* The side stream and the event fences of _StreamState (streaming/state.py:47-55,239-256;
 * streaming/activation.py:506-513). Streams are non-blocking at the default priority. wf_event_query returns 0
 * when the event's work is complete, 1 when not yet (the reference's event.query(), streaming/state.py:255). */
int wf_stream_create(void** stream);
int wf_stream_destroy(void* stream);
int wf_stream_synchronize(void* stream);
int wf_event_create(void** event, int timing);
int wf_event_destroy(void* event);
int wf_event_record(void* event, void* stream);
int wf_stream_wait_event(void* stream, void* event);
int wf_event_query(void* event);
int wf_event_synchronize(void* event);
int wf_event_elapsed_ms(void* start, void* end, float* ms);

/* ---------------------------------------------------------------------------------------------- GGUF files
 * The tensor table of a GGUF model file (version 2 or 3): the reference reads GGUF files through ComfyUI-GGUF /
 * gguf-py (not vendored; the files come from its tools/convert_to_gguf.py and llama.cpp's converters); these calls
 * give the SSD tier each tensor's absolute byte range so streamed blocks are read straight from the model file
 * (the role of file_block_layout / file_param_layout, core/tiers/plan.py:181-250, for GGUF instead of
 * safetensors). The file is untrusted: a malformed header is WF_EINVAL with a message, never a read out of
 * bounds. dims4: the tensor's dimensions, innermost first (GGUF order), padded with 1. Types: the GGML ids of
 * weightferry's formats plus F32 0, F16 1, BF16 30. */
int wf_gguf_open(const char* path, void** handle);
int wf_gguf_close(void* handle);
int wf_gguf_info(void* handle, int* version, int64_t* n_tensors, int64_t* n_kv, int64_t* alignment,
                 int64_t* data_offset, int64_t* file_bytes);
int wf_gguf_tensor(void* handle, int64_t i, char* name, int64_t name_cap, int* type, int* n_dims, int64_t* dims4,
                   int64_t* offset, int64_t* nbytes);
/* key/value i: type = GGUF value type (0-12); for arrays (9) elem_type and count; integers and bools in ival, floats
 * in fval (integers too), strings in sval (count = its length). */
int wf_gguf_kv(void* handle, int64_t i, char* key, int64_t key_cap, int* type, int* elem_type, int64_t* count,
               int64_t* ival, double* fval, char* sval, int64_t sval_cap);

/* ---------------------------------------------------------------------------------------------- SSD tier
 * A ring of `depth` host buffers filled by `threads` reader threads with streamed blocks read from the file at
 * `path`, in cyclic block order: the role of DiskRing (core/tiers/sources.py:165-355) with FileBlockSource /
 * PieceFileSource (:87-152), and, with wf_ring_submit / wf_ring_wait, of _SsdUploader (streaming/ssd_uploader.py:
 * 17-120). Block b is pieces piece_start[b] .. piece_start[b+1]-1: (file offset, bytes, offset in the packed block),
 * in increasing block offset. Flags: WF_RING_PINNED (page-locked buffers; required for submit), WF_RING_DIRECT
 * (O_DIRECT reads of 4 KiB aligned supersets through an aligned scratch buffer; ordinary reads where the file system
 * refuses). Consumers take blocks in the ring's order (block = position % n_blocks), either with acquire / release
 * from one thread (release's stream, if not NULL, must carry the copy out of the buffer: the buffer is refilled
 * after it), or with submit / wait: an uploader thread waits for the block, makes `stream` wait for `wait_event`,
 * copies into dst (dst_bytes >= the block), records `done_event` and returns the buffer to the readers; wait(ticket)
 * returns once that copy is on the stream (done_event recorded). A read or copy failure fails the ring: blocks read
 * before it are still served, later ones return an error until wf_ring_resync, which restarts the cycle at block 0
 * (no copies pending). */
#define WF_RING_PINNED 1
#define WF_RING_DIRECT 2
int wf_ring_open(const char* path, int64_t n_blocks, const int64_t* piece_start, const int64_t* piece_off,
                 const int64_t* piece_len, const int64_t* piece_dst, int depth, int threads, int flags, int device,
                 void** ring);
int wf_ring_acquire(void* ring, int64_t block, void** ptr, int64_t* nbytes, int* slot);
int wf_ring_release(void* ring, int slot, void* stream);
int wf_ring_submit(void* ring, int64_t block, void* dst, int64_t dst_bytes, void* wait_event, void* done_event,
                   void* stream, int64_t* ticket);
int wf_ring_wait(void* ring, int64_t ticket);
int wf_ring_resync(void* ring);
int wf_ring_stats(void* ring, double* read_s, double* wait_s, int64_t* bytes, int64_t* reads);
int wf_ring_close(void* ring);


#ifdef __cplusplus
}
#endif

#endif /* WEIGHTFERRY_H */
