/*
 * cacheir_hip.h -- C ABI of the MI355X (gfx950) decode-step backend for CacheIR.
 *
 * Conventions (modelled on the reference's only C-ABI kernel boundary,
 * cpp/src/cacheir_cuda_kernels.cu:273-411):
 *   - every entry point returns an int status: 0 (hipSuccess) or a hipError_t
 *     value; argument errors return hipErrorInvalidValue (1) and set the text
 *     returned by cir_last_error_string();
 *   - all pointers are device pointers owned by the caller; nothing is allocated
 *     or freed inside the library; scratch memory is passed in as `workspace`
 *     with its size from the matching *_workspace_bytes() call;
 *   - work is enqueued asynchronously on the given stream (a hipStream_t passed as
 *     void*; NULL = legacy default stream) and is stream-ordered;
 *   - empty problems (batch == 0, n == 0, ...) return 0 without launching;
 *   - the library keeps no per-call global state and is safe to call from several
 *     host threads on different streams.
 *
 * Dtype codes: CIR_F32 = 0, CIR_F16 = 1.  Weight formats use GGML type ids:
 * CIR_Q4_0 = 2, CIR_Q8_0 = 8; the reference's own per-row asymmetric int4 / int8
 * packing is CIR_I4_ROW = 64 / CIR_I8_ROW = 65.
 */
#ifndef CACHEIR_HIP_H
#define CACHEIR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CIR_F32 0
#define CIR_F16 1
#define CIR_Q4_0 2
#define CIR_Q8_0 8
/* Per-row asymmetric formats of the reference (cacheir/quantization.py:96-139,
 * PackedQuantizedTensor with axis 1): w = (q - zero_point[row]) * scale[row], q in
 * [0, 15] (4 bit) or [0, 255] (8 bit). */
#define CIR_I4_ROW 64
#define CIR_I8_ROW 65

/* Library identity and diagnostics. */
const char* cir_version(void);
const char* cir_last_error_string(void);

/* ---------------------------------------------------------------- attention ---
 * Replaces the reference's batched paged decode attention:
 *   cacheir/backends/triton_kernels.py:174-217 (paged_attention_decode_batch_kernel),
 *   driven by cacheir/runtime/cuda.py:1183-1253 (_try_triton_decode_attention_batch),
 *   C-ABI analogue cpp/src/cacheir_cuda_kernels.cu:357-411.
 * q        [batch, num_heads, head_dim]           (kv_dtype)
 * k_pool   [slots, num_kv_heads, page_size, head_dim] (kv_dtype), v_pool likewise
 * page_table [batch, max_pages] int32 slot ids; seq_lens [batch] int32 (tokens to
 *   attend, the new token included); out [batch, num_heads, head_dim] (kv_dtype).
 *   Both live on the device and are not read by the host: every entry a sequence
 *   uses (the first ceil(seq_len / page_size)) must be a slot of the pools, and
 *   seq_len at most max_pages * page_size (longer contexts are clamped to it).  The
 *   Python wrappers check this on request (check_tables=True); the runtime builds
 *   its tables from its own allocator.
 * Head h reads KV head h / (num_heads / num_kv_heads).  scale multiplies q.k
 * (the reference uses 1/sqrt(head_dim)).  A sequence with seq_len 0 yields zeros.
 * fp16 path: head_dim 128 (MFMA); fp32 path: any head_dim <= 256. */
size_t cir_paged_attention_workspace_bytes(int rows, int num_heads, int head_dim, int max_context);
int cir_paged_decode_attention(const void* q, const void* k_pool, const void* v_pool,
                               const int32_t* page_table, const int32_t* seq_lens, void* out,
                               void* workspace, size_t workspace_bytes,
                               int batch, int num_heads, int num_kv_heads, int head_dim,
                               int page_size, int max_pages, float scale, int kv_dtype, void* stream);

/* cir_paged_decode_attention without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  It allocates nothing: the split
 * partials go to a static device array of CIR_ATTENTION_NOALLOC_MAX_BYTES per GPU,
 * looked up on the first call on each device (make the stream's device current).
 * Sizes whose partials, rows * num_heads * S * (head_dim + 2) * 4 bytes with S the
 * split count, exceed it return hipErrorInvalidValue before launching (the fp16
 * head_dim-128 path never splits beyond 256 workgroups, so it fits at any batch; the
 * generic path needs 4 * num_heads * (head_dim + 2) bytes per 128 tokens per row).
 * Results are bitwise those of cir_paged_decode_attention.  Every call on one GPU
 * shares the array: calls that overlap on one GPU (two streams, two host threads)
 * race and must be serialised by the caller.  Nothing in the array needs clearing:
 * each launch writes every partial it reads. */
#define CIR_ATTENTION_NOALLOC_MAX_BYTES ((size_t)16 << 20)
int cir_paged_decode_attention_noalloc(const void* q, const void* k_pool, const void* v_pool,
                                       const int32_t* page_table, const int32_t* seq_lens, void* out,
                                       int batch, int num_heads, int num_kv_heads, int head_dim,
                                       int page_size, int max_pages, float scale, int kv_dtype, void* stream);

/* Decode attention fused with the QKV epilogue: instead of a finished q it takes the
 * QKV projection's fp32 split-k partials [splits][batch][(num_heads + 2 num_kv_heads)
 * head_dim] (q | k | v columns, as cir_qgemm writes them), applies interleaved RoPE
 * at positions[batch] to q and k (inv_freq[head_dim/2] fp32), appends k and v of the
 * new token to its page, and attends as cir_paged_decode_attention does (seq_lens
 * count the new token).  Results, including the pool contents, are bitwise those of
 * cir_epilogue_qkv_rope_append followed by cir_paged_decode_attention.  fp16 pools,
 * head_dim 128, page_size a multiple of 16, num_heads/num_kv_heads <= 8.
 * Replaces the decode pair fused_rmsnorm_qkv_rope (RoPE + KV append part,
 * cacheir/runtime/cpu.py:234-249,324-340, cuda.py:800-820) -> paged_attention_decode
 * (cacheir/backends/triton_kernels.py:174-217, cuda.py:1183-1253). */
int cir_paged_decode_attention_qkv(const float* qkv_partial, int splits, const float* inv_freq,
                                   const int32_t* positions, void* k_pool, void* v_pool,
                                   const int32_t* page_table, const int32_t* seq_lens, void* out,
                                   void* workspace, size_t workspace_bytes, int batch, int num_heads,
                                   int num_kv_heads, int head_dim, int page_size, int max_pages,
                                   float scale, void* stream);

/* The number of context splits S the decode attention above uses for these sizes
 * (1: each workgroup writes the finished output).  No reference counterpart: it tells
 * a caller whether cir_paged_decode_attention_qkv_parts applies (S > 1). */
int cir_paged_decode_splits(int batch, int num_heads, int num_kv_heads, int head_dim, int page_size, int max_pages,
                            int kv_dtype);

/* cir_paged_decode_attention_qkv without its merge: the S > 1 split partials stay in
 * the workspace, O as float [batch][num_heads][S][head_dim] at its start and (max,
 * sum) as float [batch][num_heads][S][2] right after, for cir_qgemm_attn to merge
 * while it stages the O projection's input.  Pool contents as with the merged call.
 * Same replaced pair as cir_paged_decode_attention_qkv; the merge itself is the last
 * step of the reference's attention (cacheir/backends/triton_kernels.py:174-217). */
int cir_paged_decode_attention_qkv_parts(const float* qkv_partial, int splits, const float* inv_freq,
                                         const int32_t* positions, void* k_pool, void* v_pool,
                                         const int32_t* page_table, const int32_t* seq_lens, void* workspace,
                                         size_t workspace_bytes, int batch, int num_heads, int num_kv_heads,
                                         int head_dim, int page_size, int max_pages, float scale, void* stream);

/* Causal prefill over the same paged pool (reference prefill attention semantics,
 * cacheir/runtime/cpu.py:361-368): q is [batch * q_len, num_heads, head_dim]; row
 * (b, s) attends to tokens t < seq_lens[b] - q_len + s + 1, where seq_lens[b] is the
 * length after the q_len new tokens were appended.  On the fp16 head_dim-128 path
 * (q_len > 1) the workspace is checked but not written: 128 query vectors of a sequence
 * share each K/V block read and the output is written directly. */
int cir_paged_prefill_attention(const void* q, const void* k_pool, const void* v_pool,
                                const int32_t* page_table, const int32_t* seq_lens, void* out,
                                void* workspace, size_t workspace_bytes,
                                int batch, int q_len, int num_heads, int num_kv_heads, int head_dim,
                                int page_size, int max_pages, float scale, int kv_dtype, void* stream);

/* ------------------------------------------------------------ block weights ---
 * GGUF Q4_0 / Q8_0 blocks (cacheir/importers/gguf.py:36,40,273-310) for a weight
 * W[n, k] stored row-major, blocks along k.  The GEMM reads a tiled copy made once
 * at load by cir_qweight_repack: nibbles/bytes regrouped into 16-row x 128-column
 * tiles so one wavefront load is 1 KiB contiguous, and the fp16 scales in a
 * parallel tile array.  Values are unchanged: the tiled copy dequantizes to the
 * same (q - 8) * d (Q4_0) or q * d (Q8_0) as the GGUF blocks. */
size_t cir_qweight_tiled_bytes(int fmt, int n, int k);
int cir_qweight_repack(const void* gguf_blocks, void* tiled, int fmt, int n, int k, void* stream);

/* The reference's own per-row asymmetric packing (cacheir/quantization.py:96-139,
 * PackedQuantizedTensor produced for --quant int4 / int4_awq / gptq / int8 and
 * consumed by cacheir/runtime/cuda.py:77-105,932-954) -> the tiled copy cir_qgemm
 * reads (fmt CIR_I4_ROW or CIR_I8_ROW, cir_qweight_tiled_bytes bytes).
 * packed: uint8 [n][ceil(k/2)] (4 bit: column 2j in the low nibble of byte j, 2j+1 in
 * the high nibble) or [n][k] (8 bit); scales fp32 [n]; zero_points int32 [n].
 * cir_dequant(tiled = 1) then gives exactly (q - zero_point) * scale in fp32, and
 * cir_qgemm multiplies the exact integer codes, applying scale and zero point per row
 * after the k-sum. */
int cir_qweight_repack_rows(const void* packed, const float* scales, const int32_t* zero_points, void* tiled,
                            int fmt, int n, int k, void* stream);

/* Bit-exact dequantization to fp32 [n, k] from GGUF blocks (tiled = 0) or from the
 * tiled copy (tiled = 1).  Replaces gguf.py:273-310 for device-resident weights. */
int cir_dequant(const void* weights, int tiled, int fmt, float* out, int n, int k, void* stream);

/* The k-split cir_qgemm is tuned for at this shape: enough workgroups to fill the GPU,
 * no more partials than that needs (for m <= 8, the split under which the GEMV gives
 * every CU the same share of the weights; on the large-m GEMM, one round of workgroups
 * over the CUs, which need not divide k/128).
 * 0 for an invalid shape.  (The reference has no k-split; this replaces its GEMM plan choice,
 * cacheir/runtime/cuda.py:956-974 _select_gemm_plan.) */
int cir_qgemm_splits(int m, int n, int k);
size_t cir_qgemm_workspace_bytes(int m, int n, int splits);
/* y_partial[split][m][n] = sum over split's k-range of x[m][k] * W[n][k]
 * (the matmul of cacheir/runtime/cuda.py:920-954 / cpu.py:291-312).
 * x: fp16 [m, k] row-major (row stride ldx elements); W tiled fmt blocks.
 * The MFMA multiplies the exact integers (q-8) (Q4_0) or q (Q8_0) in fp16 with x;
 * each 32-value block's fp32 result is scaled by its d in fp32 (exact products:
 * only summation order differs from the fp32 dequant-then-matmul).  fp32 accumulate.
 * m <= 8 with m * (k/128/splits) <= 128 runs the dequant GEMV (activations staged in
 * LDS once per workgroup, each wavefront streaming whole tiles); larger m the MFMA
 * GEMM.  For the same split both give the same partials bit for bit.
 * splits must divide k/128, except where the large-m GEMM runs (cir_qgemm_plan names
 * qgemm_xl_kernel): there split s covers quads s*ceil(k/128/splits) onward (the last
 * fewer) and any count that leaves no split empty is taken.  Requires k % 128 == 0. */
int cir_qgemm(const void* x, int ldx, const void* w_tiled, int fmt, float* y_partial,
              int m, int n, int k, int splits, void* stream);

/* Which kernel the GEMM entry points run for these sizes (a static string; "invalid"
 * for arguments the entry point would reject): op CIR_GEMM_PARTIALS = cir_qgemm with
 * `splits`, CIR_GEMM_SWIGLU = cir_qgemm_swiglu (n = 2 * inter), CIR_GEMM_ARGMAX =
 * cir_qgemm_argmax, CIR_GEMM_ATTN_MERGE = cir_qgemm_attn.  Pure host arithmetic.
 * Replaces the reference's per-shape GEMM plan record (cacheir/runtime/cuda.py:956-974
 * _select_gemm_plan, surfaced as CudaRuntime.gemm_plans, cuda.py:484,683-690). */
#define CIR_GEMM_PARTIALS 0
#define CIR_GEMM_SWIGLU 1
#define CIR_GEMM_ARGMAX 2
#define CIR_GEMM_ATTN_MERGE 3
const char* cir_qgemm_plan(int op, int fmt, int m, int n, int k, int splits);

/* The O projection of a decode step fed straight from split attention partials
 * (cir_paged_decode_attention_qkv_parts): the workgroup merges each head's S <= 8
 * partials into the fp16 attention output (the arithmetic and rounding of the attention's
 * own merge, so the same bits) while staging its activations,
 * then runs as cir_qgemm.  Block formats,
 * k = num_heads * 128, m <= 8 with m * (k/128/splits) <= 256.  Replaces the
 * attention output -> o_proj quantized matmul pair (cacheir/runtime/cuda.py:932-954). */
int cir_qgemm_attn(const float* attn_part_o, const float* attn_part_ml, int attn_splits, int num_heads,
                   const void* w_tiled, int fmt, float* y_partial, int m, int n, int k, int splits, void* stream);

/* Gate|up projection fused with SwiGLU (cacheir/runtime/cpu.py:266-279,
 * cuda.py:859-871 quantized_fused_swiglu): out[m][j] = silu(g) * u with g, u the
 * projections of x onto gate row j and up row j, fp32 accumulate, one launch, no
 * partials.  w_tiled is the tiled copy of the 2*inter rows in *interleaved* order --
 * gate rows 16c..16c+15, then up rows 16c..16c+15, for c = 0, 1, ... (make it by
 * permuting the GGUF block rows before cir_qweight_repack).  out dtype odt
 * (CIR_F16 / CIR_F32), [m][inter].  inter % 16 == 0, k % 128 == 0.  Bitwise equal to
 * cir_qgemm (splits 1) over the same tiles followed by cir_epilogue_swiglu. */
int cir_qgemm_swiglu(const void* x, int ldx, const void* w_tiled, int fmt, void* out, int odt, int m,
                     int inter, int k, void* stream);

/* Dense weights W[n][k] in fp32 (x fp32) -- the fp32 parity path for unquantized
 * artifacts.  Writes y_partial[split][m][n]; splits must divide ceil(k/256). */
int cir_gemm_f32(const float* x, int ldx, const float* w, float* y_partial,
                 int m, int n, int k, int splits, void* stream);

/* ---------------------------------------------------------------- epilogues ---
 * All epilogues first sum y_partial over `splits`. */

/* out[m][n] = sum + (residual ? residual[m][n] : 0).  out/residual dtype odt.
 * Residual add = graph op "add" (cpu.py:256-257) fused behind o_proj / down_proj. */
int cir_epilogue_store(const float* y_partial, int splits, const void* residual, void* out, int odt,
                       int m, int n, void* stream);

/* Residual epilogue fused with the RMSNorm that consumes its result (graph ops
 * "add" + "rms_norm", cpu.py:256-257,284-289): h = residual + sum of partials is
 * written to h_out (fp32) and xn = (h * 1/sqrt(mean(h^2) + eps)) * norm_w (dtype
 * xdt) is written for the next GEMM.  Rows up to 8192. */
int cir_epilogue_residual_rmsnorm(const float* y_partial, int splits, const float* residual, float* h_out,
                                  const void* norm_w, int wdt, float eps, void* xn, int xdt, int m, int n, void* stream);

/* SwiGLU (cpu.py:266-279): y_partial columns [0, inter) are gate, [inter, 2*inter)
 * up; out[m][j] = silu(gate) * up, dtype odt. */
int cir_epilogue_swiglu(const float* y_partial, int splits, void* out, int odt, int m, int inter, void* stream);

/* QKV epilogue of fused_rmsnorm_qkv_rope (cpu.py:234-249, RoPE cpu.py:324-340) with
 * the KV append of the attention node (cpu.py:352 / cuda.py:1218) fused in.
 * y_partial columns: [0, Hq*D) q, then Hkv*D k, then Hkv*D v.  Row r = b*q_len + s
 * is at position positions[b] + s.  Interleaved RoPE with inv_freq[D/2] (fp32,
 * computed by the caller exactly as the reference does).  q_out [rows, Hq*D] (odt);
 * k/v rows are written into k_pool/v_pool (kv dtype kvt) at slot
 * page_table[b][pos / page_size], offset pos % page_size. */
int cir_epilogue_qkv_rope_append(const float* y_partial, int splits, const float* inv_freq,
                                 const int32_t* positions, const int32_t* page_table, int max_pages,
                                 void* q_out, int odt, void* k_pool, void* v_pool, int kvt,
                                 int batch, int q_len, int num_heads, int num_kv_heads, int head_dim,
                                 int page_size, void* stream);

/* ------------------------------------------------------------- row kernels ---
 * Token embedding gather (cpu.py:223-224): out[r][:] = table[ids[r]][:]; table
 * dtype tdt, out dtype odt; ids int64.  The ids live on the device, so the call
 * cannot reject them: an id outside [0, vocab) reads row 0 or vocab - 1.  Callers
 * validate ids on the host (the runtime raises IndexError, as the reference's
 * table lookup does). */
int cir_embedding(const int64_t* ids, const void* table, int tdt, void* out, int odt,
                  int rows, int hidden, int vocab, void* stream);

/* RMSNorm (cpu.py:284-289): out = (x * 1/sqrt(mean(x^2) + eps)) * w.  x dtype xdt,
 * w dtype wdt, out dtype odt; rows of length hidden. */
int cir_rmsnorm(const void* x, int xdt, const void* w, int wdt, void* out, int odt,
                int rows, int hidden, float eps, void* stream);

/* out = a + b elementwise (graph op "add"), all of dtype dt. */
int cir_add(const void* a, const void* b, void* out, int dt, size_t count, void* stream);

/* out = in converted between dtypes (idt -> odt); count elements. */
int cir_cast(const void* in, int idt, void* out, int odt, size_t count, void* stream);

/* Greedy sampling (cpu.py:181-182, scheduler.py:535-543): ids[r] = first index of
 * the maximum of logits[r][0:vocab] (fp32, row stride ld); NaN counts as the maximum,
 * as in numpy's argmax. */
int cir_argmax(const float* logits, int ld, int64_t* ids, int rows, int vocab, void* stream);

/* LM head + greedy sampling in one pass (the lm_head matmul of cuda.py:851-852 /
 * cpu.py:256-257 followed by the argmax of scheduler.py:535-543): ids[r] = argmax over
 * j < n of (x[r] . W[j]) for the tiled weight W [n, k], without storing the logits.
 * The logits are computed exactly as cir_qgemm with splits = 1 computes them, so the
 * ids equal cir_argmax over that GEMM's output.  workspace: caller-owned device memory
 * of cir_qgemm_argmax_workspace_bytes(m, n) bytes for per-wavefront candidates. */
size_t cir_qgemm_argmax_workspace_bytes(int m, int n);
int cir_qgemm_argmax(const void* x, int ldx, const void* w_tiled, int fmt, int64_t* ids, void* workspace,
                     size_t ws_bytes, int m, int n, int k, void* stream);

/* ------------------------------------------------------------- calibration ---
 * Reads `bytes` (a multiple of 16) from buf with `workgroups` x `threads` threads,
 * grid-stride (layout 0) or one contiguous chunk per workgroup (layout 1), and writes
 * nothing but an unreachable sentinel to out (one uint32).  With side_ratio 1..8 each
 * thread also reads side_ratio 16-byte chunks of `side` (side_bytes, a power of two of
 * 16-byte chunks, small enough to stay in L2) per 8 chunks of buf, issued together:
 * the load pattern of a GEMM that streams weights and re-reads activations.  No
 * counterpart in the reference: it measures what a plain read of a hot kernel's bytes
 * reaches on this GPU, the ceiling the roofline fractions are read against. */
int cir_stream_read(const void* buf, size_t bytes, int workgroups, int threads, int layout, const void* side,
                    size_t side_bytes, int side_ratio, void* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* CACHEIR_HIP_H */
