/*
 * mle_hip.h -- C ABI of the MI355X (gfx950) backward / optimizer hot path.
 *
 * This is the boundary that replaces the `<<<...>>>` call sites inside the
 * GraphOperations lambdas of ML_Engine (Engine/engine.cu) and the host wrappers
 * of Includes/kernels.h.  The C++ graph layer (ml_engine_amd/engine/engine.h)
 * calls only these functions; a different host language binds the same symbols.
 *
 * Conventions
 *  - Every function returns int: 0 = MLE_OK, < 0 = an mle_status.  The message
 *    of the last failure on the calling thread is returned by mle_last_error().
 *  - Tensors are plain device pointers to fp32 (int32 for token ids), row-major,
 *    with the reference's [batch, channels, rows, cols] layout.
 *  - Calls enqueue work on `stream` (a hipStream_t; NULL = the null stream) and
 *    never synchronise, except mle_stream_sync, the mle_memcpy_h2d/d2h helpers
 *    (which wait for their own copy) and mle_probe_read.
 *  - Calls never allocate device memory, except mle_device_alloc and the arena
 *    calls.  Kernels that need scratch take (ws, ws_bytes); the required size is
 *    returned by the matching *_ws_bytes query.
 *  - "accumulate" means the kernel adds into its destination (`+=`), as the
 *    reference backward kernels do; "assign" overwrites.  Backward entry points
 *    that take `int accumulate` do either: 1 is the reference's `+=`, 0 writes
 *    the value that `+=` would leave in a zeroed destination without reading
 *    it (callers use it for the first write after zero_grad).
 */
#ifndef MLE_HIP_H
#define MLE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mle_stream;              /* hipStream_t */
typedef struct mle_arena_s* mle_arena; /* bump allocator over one device buffer */

enum mle_status {
  MLE_OK = 0,
  MLE_ERR_INVALID = -1,     /* bad shape / argument (reference: print + exit) */
  MLE_ERR_HIP = -2,         /* HIP runtime error (reference: CheckError)       */
  MLE_ERR_OOM = -3,         /* allocation failed (reference: SafeCudaMalloc)   */
  MLE_ERR_UNSUPPORTED = -4, /* shape outside what a kernel supports           */
  MLE_ERR_WORKSPACE = -5    /* workspace smaller than *_ws_bytes reported      */
};

enum mle_act_kind { MLE_RELU = 0, MLE_GELU = 1, MLE_SILU = 2, MLE_TANH = 3, MLE_SIGMOID = 4, MLE_LEAKY_RELU = 5 };

/* ------------------------------------------------------------------------- */
/* Runtime: errors, device memory, streams, arena                            */
/* ------------------------------------------------------------------------- */

/* Message of the last failed call on this thread ("" if none). */
const char* mle_last_error(void);
/* Library version string, e.g. "mle_hip 0.1 gfx950". */
const char* mle_version(void);
/* Make `device` current and check that it is gfx950.  Replaces the implicit
 * CUDA context creation of the reference. */
int mle_init(int device);

/* Device allocation.  Replaces SafeCudaMalloc (Includes/debugging_utils.h:98-110):
 * returns MLE_ERR_OOM with the free/total memory in the message. */
int mle_device_alloc(void** ptr, size_t bytes);
int mle_device_free(void* ptr);
int mle_memcpy_h2d(void* dst, const void* src, size_t bytes, mle_stream stream);
/* Synchronous device-to-host copy (ReadValueAt, Engine/engine.cu:3-9). */
int mle_memcpy_d2h(void* dst, const void* src, size_t bytes, mle_stream stream);
/* Reads one float from device memory once the work queued on `stream` before
 * it has run: the loss read-back of the loss nodes' forward (cudaMemcpy(&loss,
 * node->output, ...), Engine/engine.cu:1656,1700,1935,2046,2098).  A one-thread
 * kernel publishes the value and a sequence number into pinned host memory and
 * the caller spins on the sequence number, so it resumes as soon as the value
 * lands instead of waking from a blocking wait.  Calls on one device are
 * serialised. */
int mle_read_scalar(mle_stream stream, const float* src, float* dst);
/* The value the last mle_read_scalar on this device published (after the
 * caller synchronised the stream): under graph capture mle_read_scalar only
 * records its publishing kernel, and each replay of the graph publishes. */
int mle_scalar_last(float* dst);
/* The slot's state on the current device: the last published value and its
 * sequence number, and the last sequence number handed out.  A recorded graph
 * publishes, on every replay, the number its mle_read_scalar was given at
 * capture; a caller that noted it can tell whether the slot still holds its
 * own graph's value (any value or pointer may be null). */
int mle_scalar_state(float* value, unsigned* published, unsigned* issued);
/* Mark the slot empty (published sequence number 0), and wait -- spinning,
 * like mle_read_scalar -- until the last number published is `seq`, then
 * return the value.  A caller that replays a recorded graph (which publishes
 * the same number on every replay) clears the slot before the launch and
 * reads the loss as soon as the replay publishes it, instead of after the
 * stream drains.  expect fails (MLE_ERR_INVALID) when the stream drains
 * without `seq` being the last number published. */
int mle_scalar_clear(void);
int mle_scalar_expect(mle_stream stream, unsigned seq, float* dst);

/* Graphs.  The work a caller enqueues on `stream` between capture_begin and
 * capture_end is recorded (not run) into a graph, instantiated once;
 * mle_graph_launch replays it with one launch.  The engine records its
 * zero_grad -> forward -> backward pass this way (mle_model_step_graph): the
 * kernels and their arguments are fixed at capture, so a replay computes on
 * whatever the captured buffers hold when it runs.  No reference
 * counterpart: the reference launches every kernel from the host each step. */
typedef struct mle_graph_s* mle_graph;
int mle_graph_capture_begin(mle_stream stream);
int mle_graph_capture_end(mle_stream stream, mle_graph* out);
int mle_graph_launch(mle_graph graph, mle_stream stream);
int mle_graph_destroy(mle_graph graph);
int mle_memcpy_d2d(void* dst, const void* src, size_t bytes, mle_stream stream);

int mle_stream_create(mle_stream* stream);
int mle_stream_destroy(mle_stream stream);
/* Wait for the stream; reports asynchronous kernel faults like CheckError
 * (Engine/debug.cu:15-25). */
int mle_stream_sync(mle_stream stream);

/* Static arena: one device buffer, 256-byte aligned bump allocation.  Replaces
 * the per-node cudaMalloc of NodeBackProp (Engine/engine.cu:45-64). */
int mle_arena_create(size_t bytes, mle_arena* arena);
int mle_arena_alloc(mle_arena arena, size_t bytes, void** ptr);
int mle_arena_reset(mle_arena arena);
int mle_arena_destroy(mle_arena arena);
size_t mle_arena_used(mle_arena arena);
size_t mle_arena_capacity(mle_arena arena);

/* ------------------------------------------------------------------------- */
/* Elementwise / data movement                                               */
/* ------------------------------------------------------------------------- */

/* x[i] = value.  fillKernel (Includes/kernels.h:13-19), Zerograd (Engine/engine.cu:312-326). */
int mle_fill(mle_stream stream, float* x, float value, size_t n);
/* z = x + scale*y.  ScaleAdd (Engine/kernels.cu:1718-1724). */
int mle_scale_add(mle_stream stream, const float* x, const float* y, float* z, float scale, size_t n);
/* y += scale*x (double scale, float storage).  Accumulate (Engine/kernels.cu:1693-1699). */
int mle_accumulate(mle_stream stream, const float* x, float* y, double scale, size_t n);
/* y = (float)(scale*(double)x): mle_accumulate into a zeroed y, without reading y. */
int mle_scale_assign(mle_stream stream, const float* x, float* y, double scale, size_t n);
/* Both gradients of an Add at once: ya (+)= x and yb (+)= x in one pass over x
 * (acc_* == 0 assigns).  Equals mle_accumulate / mle_scale_assign at scale 1 on
 * each destination.  Add backward (Engine/engine.cu:1630-1672): its two
 * Accumulate launches (Engine/kernels.cu:1693-1699).  ya and yb must differ. */
int mle_accumulate2(mle_stream stream, const float* x, float* ya, int acc_a, float* yb, int acc_b, size_t n);
/* The residual Add and the activation after it (out = SILU(Add(h, skip)) in
 * the residual block, Engine/diffusion.cu:129-137; Add, Engine/engine.cu:
 * 1630-1672):
 *   mle_add_act_fwd: z = a + b and y = act(z) in one pass.
 *   mle_act_bwd_add: dz (+)= act'(z) * da (accumulate_dz 1 adds), then
 *     ga (+)= dz and gb (+)= dz (acc_a / acc_b) in one pass.
 * The same bits as mle_scale_add + mle_act_fwd, and mle_act_bwd +
 * mle_accumulate2. */
int mle_add_act_fwd(mle_stream stream, const float* a, const float* b, float* z, float* y, int kind, size_t n);
int mle_act_bwd_add(mle_stream stream, const float* z, const float* da, int kind, float* dz, int accumulate_dz,
                    float* ga, int acc_a, float* gb, int acc_b, size_t n);
/* y = scale*x.  Scale_Write (Engine/kernels.cu:1677-1682), Write (Engine/kernels.cu:1670-1675) with scale 1. */
int mle_scale_write(mle_stream stream, const float* x, float* y, float scale, size_t n);
/* divide==0: x *= factor; divide==1: x /= factor.  SV (Includes/kernels.h:272-280). */
int mle_scale_inplace(mle_stream stream, float* x, float factor, int divide, size_t n);
/* x *= (float)s[0] or x /= (float)s[0] with s a device double.  SP (Includes/kernels.h:293-300). */
int mle_scale_by_device(mle_stream stream, float* x, const double* s, int divide, size_t n);
/* y[r, :] += b[:] for r < rows.  BCumAdd (Engine/kernels.cu:1586-1592). */
int mle_bias_add_rows(mle_stream stream, float* y, const float* b, size_t rows, int cols);
/* y = x + b[channel] over [B, C, HW].  broadcast_add (Engine/kernels.cu:1661-1668). */
int mle_broadcast_channel_add(mle_stream stream, const float* x, const float* b, float* y, int batch, int channels, size_t hw);
/* [B,1,S,H*D] <-> [B,H,S,D].  HeadifyColChannel (Engine/kernels.cu:1371-1406):
 * flag 0: out[headified] = in[flat]   (HeadifytoChannel forward)
 * flag 1: out[flat]     += in[headified] (HeadifytoChannel backward)
 * flag 2: out[flat]      = in[headified] (DeHeadify forward)
 * flag 3: out[headified] += in[flat]   (DeHeadify backward)
 * The accumulating flags are plain adds: every destination is written once. */
int mle_headify(mle_stream stream, const float* in, float* out, int batch, int heads, int seq, int head_dim, int flag);
/* y = x + PE, PE = sin (even dims) / cos (odd dims) of pos/10000^(2i/cols).
 * MatPEncoding (Engine/kernels.cu:166-185). */
int mle_matpe(mle_stream stream, const float* x, float* y, int batch, int rows, int cols, int start_idx);
/* pe[r, c] = sin (even c) / cos (odd c) of (start_idx + r) / 10000^(2 floor(c/2) / cols),
 * the encoding MatPEncoding adds (Engine/kernels.cu:166-185), evaluated once by
 * the same double-precision formula as mle_matpe: mle_add_broadcast(x, pe, y)
 * then gives mle_matpe's y bit for bit. */
int mle_matpe_table(mle_stream stream, float* pe, int rows, int cols, int start_idx);
/* y[b, i] = x[b, i] + t[i] for b < batch, i < n (batch <= 65535): the add of
 * MatPEncoding with its encoding precomputed by mle_matpe_table. */
int mle_add_broadcast(mle_stream stream, const float* x, const float* t, float* y, int batch, size_t n);
/* Timestep embedding: cos half then sin half.  PEncoding (Engine/kernels.cu:147-164). */
int mle_timestep_pe(mle_stream stream, float* y, int t, int dim);

/* ------------------------------------------------------------------------- */
/* Activations                                                               */
/* ------------------------------------------------------------------------- */

/* y = f(x).  ReLU/GeLU/SiLU/TaNH/Sigmoid/LeakyReLU (Engine/kernels.cu:1214-1328). */
int mle_act_fwd(mle_stream stream, int kind, const float* x, float* y, size_t n);
/* dx (+)= dy * f'(x).  deriv_* (Engine/kernels.cu:1223-1328). */
int mle_act_bwd(mle_stream stream, int kind, const float* x, const float* dy, float* dx, size_t n, int accumulate);

/* ------------------------------------------------------------------------- */
/* GEMM (fp32 MFMA)                                                          */
/* ------------------------------------------------------------------------- */

/* C[b] = alpha * op(A[b]) * op(B[b]) + beta * C[b],  b < batch, row-major.
 *   op(A) is M x K: trans_a == 0 -> A[i*lda + k],  trans_a == 1 -> A[k*lda + i]
 *   op(B) is K x N: trans_b == 0 -> B[k*ldb + j],  trans_b == 1 -> B[j*ldb + k]
 * Strides are in elements between consecutive batch items; a stride of 0
 * broadcasts that operand (the reference's batch_chan_offset flags 0-2,
 * Engine/kernels.cu:371-385).  beta == 0 assigns (bcmm*, backward == 0),
 * beta == 1 accumulates (backward == 1, which the reference does with atomicAdd).
 * If colsum != NULL (batch == 1 only) the kernel also adds column sums of op(B)
 * over K into colsum[N] -- the Linear bias gradient fused into the dW pass
 * (BCompress, Engine/kernels.cu:1562-1584).
 * Replaces bcmm / bcmmABT / bcmmATB / bcmmT (Engine/kernels.cu:387-539). */
int mle_gemm(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha,
             const float* A, int64_t lda, int64_t stride_a,
             const float* B, int64_t ldb, int64_t stride_b, float beta,
             float* C, int64_t ldc, int64_t stride_c, int batch, float* colsum);

/* Workspace that lets mle_gemm_ex split K across workgroups when the tile grid
 * alone would leave most CUs idle (0 when no split is used for this shape; a
 * small product that runs on one of the small-product kernels, K split over
 * a workgroup's waves, leaves it unused). */
size_t mle_gemm_ws_bytes(int M, int N, int K, int batch);
/* mle_gemm plus two fusions:
 *   bias (nullable): C[b][r, c] += bias[c] after alpha/beta -- the Linear
 *     forward's BCumAdd (Engine/kernels.cu:1586-1592) in the GEMM epilogue;
 *   ws (nullable): split K over workgroups; partial tiles are summed in split
 *     order, so results are deterministic for a given shape. */
int mle_gemm_ex(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha,
                const float* A, int64_t lda, int64_t stride_a,
                const float* B, int64_t ldb, int64_t stride_b, float beta,
                float* C, int64_t ldc, int64_t stride_c, int batch, float* colsum,
                const float* bias, void* ws, size_t ws_bytes);

/* mle_gemm_ex over a batch with a bias and a fused column sum per item:
 * item b adds bias + b*stride_bias and accumulates its column sums of op(B)
 * into colsum + b*stride_colsum.  Several Linear layers that read the same
 * input (attention's Q, K and V projections, Engine/transformer.cu:650-652)
 * run as one launch: their forward (A broadcast with stride_a 0) and their
 * dW + db (Linear backward, Engine/engine.cu:3553-3560). */
int mle_gemm_batched_ex(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha,
                        const float* A, int64_t lda, int64_t stride_a,
                        const float* B, int64_t ldb, int64_t stride_b, float beta,
                        float* C, int64_t ldc, int64_t stride_c, int batch,
                        float* colsum, int64_t stride_colsum, const float* bias, int64_t stride_bias,
                        void* ws, size_t ws_bytes);

/* C = alpha * sum_{t < terms} op(A + t*stride_a_term) op(B + t*stride_b_term) + beta * C,
 * the terms summed in order (deterministic: on the register-direct kernel
 * they extend one K loop; otherwise each term is a split whose partial
 * products are reduced in term order).  The input gradient of several
 * Linear layers that share an input, dX = sum_t dY_t W_t^T, in one launch
 * instead of `terms` accumulating bcmmABT calls (Engine/engine.cu:3553).
 * Needs mle_gemm_sum_ws_bytes(M, N, terms) bytes of workspace. */
size_t mle_gemm_sum_ws_bytes(int M, int N, int terms);
int mle_gemm_sum(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha,
                 const float* A, int64_t lda, int64_t stride_a_term,
                 const float* B, int64_t ldb, int64_t stride_b_term, float beta,
                 float* C, int64_t ldc, int terms, void* ws, size_t ws_bytes);

/* mle_gemm_ex over a two-level batch: item (o, i), o < outer, i < inner,
 * reads A at A + o*sa_outer + i*sa_inner (likewise B, C).  With inner = heads
 * and the head stride as *_inner, the per-head products of attention address
 * Q, K, V and the output in their [batch, seq, heads * dim] layout directly:
 * it replaces HeadifytoChannel / DeHeadify (HeadifyColChannel,
 * Engine/kernels.cu:1371-1406) around the BMM / BMMABT bcmm calls of
 * MultiHeadAttention (Engine/transformer.cu:647-661).  ws as mle_gemm_ex with
 * batch = outer * inner. */
int mle_gemm_grid(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha,
                  const float* A, int64_t lda, int64_t sa_outer, int64_t sa_inner,
                  const float* B, int64_t ldb, int64_t sb_outer, int64_t sb_inner, float beta,
                  float* C, int64_t ldc, int64_t sc_outer, int64_t sc_inner, int outer, int inner,
                  void* ws, size_t ws_bytes);

/* mle_gemm_ex (one batch item) that also writes row statistics of C for a
 * following softmax cross-entropy (SoftMaxCrossEntropy, Engine/engine.cu:
 * 2064-2124, reads the logits again to find them): for row r and 64-column
 * block b, rowpart[r * ldp + 2b] = max of C over the block and [.. + 1] = sum
 * of exp(C - max).  On the persistent GEMM kernel the epilogue computes them
 * from the tile in registers; otherwise a second kernel reads C.  ldp >=
 * 2 * ceil(N / 64), even; rowpart 8-byte aligned. */
int mle_gemm_rowstats(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha,
                      const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                      float* C, int64_t ldc, const float* bias, float* rowpart, int64_t ldp,
                      void* ws, size_t ws_bytes);

/* A Linear layer and the activation after it (ReLU / GELU / SiLU / ...; the
 * RELU / GELU / SILU ops, Engine/engine.cu:2650-2780) with C and Y
 * contiguous rows of N floats (ldc = N), batch 1:
 *   mle_gemm_act_fwd:  C = alpha op(A) op(B) + beta C + bias;  Y = act(C)
 *   mle_gemm_act_bwd:  C = alpha op(A) op(B) + beta C  (the activation
 *                      output's gradient);  dX (+)= C * act'(X)  (its input's
 *                      gradient; accumulate_dx 1 adds, 0 assigns)
 * On the persistent GEMM kernel (NN forward / NT backward, ReLU, GELU or SiLU)
 * the epilogue computes Y or dX from the tile in registers; a forward split
 * along K has the reduce that completes C write Y too; otherwise the
 * activation kernels run after the GEMM.  Same values either way.  (The
 * engine uses the forward for small products only, a classifier's hidden
 * layer: on the C4 block's FFN, with two tiles per workgroup, the longer
 * epilogue measured no faster than a separate activation pass.) */
int mle_gemm_act_fwd(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha,
                     const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                     float* C, const float* bias, int kind, float* Y, void* ws, size_t ws_bytes);
int mle_gemm_act_bwd(mle_stream stream, int trans_a, int trans_b, int M, int N, int K, float alpha,
                     const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                     float* C, int kind, const float* X, float* dX, int accumulate_dx,
                     void* ws, size_t ws_bytes);

/* Linear backward (Engine/engine.cu:3553-3560: bcmmABT for dX, bcmmATB for
 * dW, BCompress for db) in as few launches as the shapes allow, for `layers`
 * Linear layers of shape in -> out that read the same X [rows, in]:
 *   dX      (+)= sum_l dY_l W_l^T      (accumulate_dx: 1 adds, 0 assigns)
 *   dW_l     += X^T dY_l
 *   db_l     += sum_rows dY_l          (db may be NULL)
 * Layer l's dY, W (and dW), db sit at l * stride_dy, l * stride_w, l * stride_db
 * floats (strides unused when layers == 1).  When both products run on the
 * register-direct GEMM at most one workgroup per CU each, or both on one of
 * the small-product kernels, they share one launch; otherwise dX then dW (a
 * weight gradient of one round of tiles beside a larger dX runs as two K
 * splits).  Needs mle_linear_bwd_ws_bytes(rows, in, out, layers) bytes of
 * workspace. */
size_t mle_linear_bwd_ws_bytes(int rows, int in, int out, int layers);
int mle_linear_bwd(mle_stream stream, int rows, int in, int out, int layers,
                   const float* X, const float* dY, int64_t stride_dy,
                   const float* W, int64_t stride_w, float* dX, int accumulate_dx,
                   float* dW, float* db, int64_t stride_db, void* ws, size_t ws_bytes);
/* mle_linear_bwd with the parameter gradients' mode: accumulate_dw 1 adds dW
 * and db as above, 0 assigns both (the gradients are logically zero: the
 * engine's lazy clearing of parameter gradients, no fill launch). */
int mle_linear_bwd_ex(mle_stream stream, int rows, int in, int out, int layers,
                      const float* X, const float* dY, int64_t stride_dy,
                      const float* W, int64_t stride_w, float* dX, int accumulate_dx,
                      float* dW, float* db, int64_t stride_db, int accumulate_dw, void* ws, size_t ws_bytes);
/* One Linear layer's backward (mle_linear_bwd_ex, layers = 1) followed by
 * the backward of the activation that produced its input X = act(act_x):
 *   act_dx (+)= act'(act_x) * dX       (act_accumulate: 1 adds, 0 assigns)
 * the derivative kernels of Engine/kernels.cu:1223, 1256, 1297 (ReLU, SiLU,
 * GELU; also tanh, sigmoid, leaky ReLU), run by the reference as the
 * activation node's own backward after the Linear's (Engine/engine.cu:3553-
 * 3560).  dX is written as mle_linear_bwd_ex writes it; act_x and act_dx are
 * [rows, in] like dX.  On the small-product kernels the activation gradient
 * is their epilogue (one launch less), otherwise a pass after the products.
 * act_dx may be act_x but none of X, dY, W, dX.  Same workspace as
 * mle_linear_bwd_ex. */
int mle_linear_bwd_act(mle_stream stream, int rows, int in, int out, const float* X, const float* dY,
                       const float* W, float* dX, int accumulate_dx, float* dW, float* db, int accumulate_dw,
                       int act_kind, const float* act_x, float* act_dx, int act_accumulate, void* ws,
                       size_t ws_bytes);

/* out[c] (+)= sum_r x[r, c].  BCompress (Engine/kernels.cu:1562-1584); beta 0/1. */
int mle_colsum(mle_stream stream, const float* x, size_t rows, int cols, float* out, float beta);
/* out[c] += sum_{b, s} x[b, c, s] for c < nreduce (nreduce <= channels).
 * Channel_Squeeze1D (Engine/kernels.cu:1734-1761); `nreduce` is the launch's
 * block count, which the reference sets to `out` in Convolute2D and to the
 * width in Broadcast_Channel (Engine/engine.cu:1435). */
int mle_channel_sum(mle_stream stream, const float* x, int batch, int channels, size_t hw, int nreduce, float* out);
/* mle_channel_sum with the destination's mode: accumulate 1 adds as above; 0
 * assigns out[c] for c < nreduce and sets out[nreduce .. out_total) to 0 (out is
 * logically zero: the engine's lazy clearing, no separate fill). */
int mle_channel_sum_ex(mle_stream stream, const float* x, int batch, int channels, size_t hw, int nreduce, float* out,
                       size_t out_total, int accumulate);

/* ------------------------------------------------------------------------- */
/* Softmax and losses                                                        */
/* ------------------------------------------------------------------------- */

/* Softmax over [BC, rows, cols].  axis 0 = along each row (type 0), axis 1 =
 * along each column (type 1).  causal: entries with col > row are 0 and the
 * max still runs over all entries of the line.  Sums below 1e-45 become 1.
 * SoftMax / SoftMask (Engine/kernels.cu:2183-2235). */
int mle_softmax_fwd(mle_stream stream, const float* x, float* y, int bc, int rows, int cols, int axis, int causal);
/* dx (+)= y * (dy - <dy, y>) along the same axis.  deriv_softmax (Engine/kernels.cu:2149-2181). */
int mle_softmax_bwd(mle_stream stream, const float* y, const float* dy, float* dx, int bc, int rows, int cols, int axis,
                    int accumulate);

/* Fused multi-head attention over [batch, seq, ld] projections (head h in
 * columns h*64 .. h*64+63; head_dim must be 64, seq a multiple of 64):
 * out_h = SOFTMASK(scale * q_h k_h^T, type 1) v_h, the column-normalised
 * softmax with the column maximum over every row and, when causal, keys after
 * the query masked out of the column sums.  Replaces HeadifytoChannel + BMMABT
 * + Scale + SOFTMASK/SOFTMAX(type 1) + BMM + DeHeadify of MultiHeadAttention
 * (Engine/transformer.cu:647-661; Engine/engine.cu:1144-1178, 2205-2314,
 * 2430-2505, 2523-2551), without storing the [seq x seq] scores.  ws
 * (mle_attention_ws_bytes) receives the column statistics the backward reads
 * and, for seq <= 256 with the causal mask, the probabilities on or below the
 * diagonal (seq/16 (seq/16 + 1)/2 blocks of 1 KB per batch item and head):
 * keep it unchanged between the two calls. */
size_t mle_attention_ws_bytes(int batch, int heads, int seq);
int mle_attention_fwd(mle_stream stream, const float* q, const float* k, const float* v, float* out, int batch,
                      int heads, int seq, int head_dim, int ld, float scale, int causal, void* ws, size_t ws_bytes);
/* Backward of mle_attention_fwd given dout: dq (+)= scale dS k, dv (+)= P^T dout,
 * dk (+)= scale dS^T q -- or, with k_reference_grad, BMMABT's reference
 * gradient bcmmT(q, dS) written row-major into each head's [seq x 64] block
 * (Engine/engine.cu:2307) -- where dS = P (dP - colsum(P dP)) is deriv_SoftMax
 * of type 1 (Engine/kernels.cu:2149-2181).  acc_*: 1 accumulates, 0 assigns. */
int mle_attention_bwd(mle_stream stream, const float* q, const float* k, const float* v, const float* dout, float* dq,
                      float* dk, float* dv, int batch, int heads, int seq, int head_dim, int ld, float scale,
                      int causal, int acc_q, int acc_k, int acc_v, int k_reference_grad, void* ws, size_t ws_bytes);

size_t mle_loss_ws_bytes(size_t n);
/* loss[0] = sum((t - x)^2) / n.  scalar_mse_kernel (Engine/kernels.cu:1808-1816). */
int mle_mse_fwd(mle_stream stream, const float* x, const float* t, size_t n, float* loss, void* ws, size_t ws_bytes);
/* mle_mse_fwd followed by mle_read_scalar(loss, loss_host) -- the last loss
 * node's forward with its read-back (Engine/engine.cu:2046): the kernel that
 * adds the partials also publishes the value (same bits as mle_mse_fwd), so
 * no publishing kernel runs.  The same locking and graph-capture behaviour
 * as mle_read_scalar. */
int mle_mse_fwd_read(mle_stream stream, const float* x, const float* t, size_t n, float* loss, void* ws,
                     size_t ws_bytes, float* loss_host);
/* mle_mse_fwd_read and, from the same pass over x and t, the last MSE node's
 * gradient dx = 2 (x - t) / n, assigned (scalar_mse_kernel and
 * deriv_mse_kernel with last = true, Engine/kernels.cu:1808-1816, 1838-1848):
 * the same bits as mle_mse_bwd(..., NULL, dx, n, 0). */
int mle_mse_fwd_bwd_read(mle_stream stream, const float* x, const float* t, size_t n, float* loss, float* dx,
                         void* ws, size_t ws_bytes, float* loss_host);
/* mle_mse_fwd_bwd_read when the prediction is an activation's output
 * x = act(z) (Engine/kernels.cu:1214, 1248, 1286 and their derivatives),
 * reading z instead of x: the loss (x recomputed from z with the
 * activation's function, the bits mle_act_fwd stores), its read-back,
 * x's gradient dx = 2 (x - t) / n and z's gradient dz = act'(z) * dx, both
 * assigned -- the bits of mle_mse_fwd_bwd_read on x followed by
 * mle_act_bwd(act_kind, z, dx, dz, n, 0), in one pass over z and t.  dx,
 * dz and t are distinct buffers; dz may be z. */
int mle_mse_act_fwd_bwd_read(mle_stream stream, const float* z, const float* t, size_t n, int act_kind, float* loss,
                             float* dx, float* dz, void* ws, size_t ws_bytes, float* loss_host);
/* mle_mse_act_fwd_bwd_read when z is an Add's output: z = a + b is formed
 * in the same pass (Add forward, Engine/engine.cu:1630-1672; the bits of
 * mle_add_act_fwd's z) and stored unless z is NULL, so the Add, the
 * activation after it and the last MSE node run as one pass over a, b and
 * t.  z (when set), dx and dz are distinct and alias none of a, b and t. */
int mle_add_mse_act_fwd_bwd_read(mle_stream stream, const float* a, const float* b, float* z, const float* t,
                                 size_t n, int act_kind, float* loss, float* dx, float* dz, void* ws, size_t ws_bytes,
                                 float* loss_host);
/* dx (+)= 2 (x - t) / n * (upstream ? upstream[0] : 1).  deriv_mse_kernel (Engine/kernels.cu:1838-1848). */
int mle_mse_bwd(mle_stream stream, const float* x, const float* t, const float* upstream, float* dx, size_t n,
                int accumulate);
/* probs = row softmax(logits) over [rows, cols]; loss[0] = sum(-t log(p + 1e-27)) / (rows*cols).
 * SoftMaxCrossEntropy forward (Engine/engine.cu:2088-2100, Engine/kernels.cu:1818-1826). */
int mle_softmax_xent_fwd(mle_stream stream, const float* logits, const float* target, float* probs,
                         int rows, int cols, float* loss, void* ws, size_t ws_bytes);
/* dlogits = (probs - t) * (upstream ? upstream[0] : 1) / batch  (assign).
 * SoftMaxCrossEntropy backward (Engine/engine.cu:2104-2110). */
int mle_softmax_xent_bwd(mle_stream stream, const float* probs, const float* target, const float* upstream,
                         float* dlogits, size_t n, int batch);

/* SoftMaxCrossEntropy against key targets for small logits (rows <= 1024,
 * cols <= 64, e.g. a classifier head) in one launch: the row statistics
 * (stats), the loss and (loss_host non-null) its read-back, and with dlogits
 * non-null the gradient (p - t) / batch, assigned -- the same bits as
 * mle_gemm_rowstats' row statistics, mle_softmax_xent_keys_fwd_rowstats_read
 * and mle_softmax_xent_keys_bwd (Engine/engine.cu:2088-2110). */
int mle_softmax_xent_keys_small_read(mle_stream stream, const float* logits, const int32_t* keys, int clen,
                                     int max_clen, float* stats, int rows, int cols, int batch, float* loss,
                                     float* dlogits, float* loss_host);
/* A classifier head -- Linear (logits = X W + bias, Engine/engine.cu:3505-3530)
 * followed by SoftMaxCrossEntropy against key targets (Engine/engine.cu:
 * 2088-2110) -- in one launch when the logits are at most 16 tiles of 16 x 16
 * and 4096 values (else mle_gemm_ex then mle_softmax_xent_keys_small_read):
 * logits [rows, cols] are written, then everything
 * mle_softmax_xent_keys_small_read does with them (the same bits for the
 * same logits; the logits' products are added in this kernel's own order).
 * X [rows, in], W [in, cols], bias [cols] or NULL; rows <= 1024, cols <= 64;
 * logits is a buffer of its own (not X, W or dlogits). */
int mle_linear_xent_keys_small_read(mle_stream stream, int rows, int in, int cols, const float* X, const float* W,
                                    const float* bias, float* logits, const int32_t* keys, int clen, int max_clen,
                                    float* stats, int batch, float* loss, float* dlogits, float* loss_host);
/* Cross-entropy against one-hot rows given by token ids: row r = b*clen + s
 * has its 1 at column keys[b*max_clen + s] if that id is in [0, cols), else
 * no 1 -- the matrix OneHotEmbeddings builds (Engine/kernels.cu:1551-1560).
 * Forward writes the loss (as mle_softmax_xent_fwd, bit for bit) and each
 * row's (max, sum) to stats[rows][2] instead of the probabilities; backward
 * assigns dlogits = (p - t) * (upstream ? upstream[0] : 1) / batch with p
 * recomputed from logits and stats (as mle_softmax_xent_bwd, bit for bit). */
int mle_softmax_xent_keys_fwd(mle_stream stream, const float* logits, const int32_t* keys, int clen, int max_clen,
                              float* stats, int rows, int cols, float* loss, void* ws, size_t ws_bytes);
int mle_softmax_xent_keys_bwd(mle_stream stream, const float* logits, const float* stats, const int32_t* keys,
                              int clen, int max_clen, const float* upstream, float* dlogits, int rows, int cols,
                              int batch);
/* mle_softmax_xent_keys_fwd from row statistics instead of the logits: rowpart
 * holds, per row r and 64-column block b, the block's max and sum of
 * exp(x - max) at rowpart[r * ldp + 2b], [.. + 1] (mle_gemm_rowstats writes
 * them with the logits).  The pairs combine into the row max and sum the
 * backward reads from `stats`; only the key's logit is read.  Same loss and
 * stats as mle_softmax_xent_keys_fwd up to float summation order. */
int mle_softmax_xent_keys_fwd_rowstats(mle_stream stream, const float* logits, const float* rowpart, int64_t ldp,
                                       const int32_t* keys, int clen, int max_clen, float* stats, int rows, int cols,
                                       float* loss, void* ws, size_t ws_bytes);
/* mle_softmax_xent_keys_fwd_rowstats followed by mle_read_scalar(loss,
 * loss_host) -- the cross-entropy node's forward with its read-back
 * (Engine/engine.cu:2098) -- as mle_mse_fwd_read does: same loss bits and
 * stats, no publishing kernel. */
int mle_softmax_xent_keys_fwd_rowstats_read(mle_stream stream, const float* logits, const float* rowpart,
                                            int64_t ldp, const int32_t* keys, int clen, int max_clen, float* stats,
                                            int rows, int cols, float* loss, void* ws, size_t ws_bytes,
                                            float* loss_host);

/* ------------------------------------------------------------------------- */
/* Normalisation (gamma = 1, beta = 0, as the reference)                     */
/* ------------------------------------------------------------------------- */

/* Statistics over each (batch item, group): groups == 1 is LayerNorm over the
 * whole C*H*W sample (LayerMean/LayerStd/LNorm, Engine/kernels.cu:541-572,
 * 670-699, 794-804); groups > 1 is GroupNorm (GroupMean/GroupStd/GNorm,
 * Engine/kernels.cu:607-639, 732-763, 818-834).
 * stats[2*g] = mean, stats[2*g+1] = sum of squared deviations (the reference's
 * `std` array).  y = (x - mean) * rsqrt(ssd / N + eps). */
size_t mle_norm_ws_bytes(int batch, int channels, size_t hw, int groups);
int mle_norm_fwd(mle_stream stream, const float* x, float* y, float* stats,
                 int batch, int channels, size_t hw, int groups, float eps, void* ws, size_t ws_bytes);
/* mle_norm_fwd whose first pass (per-chunk statistics of x) already ran in
 * mle_add_norm_partials on the same workspace: stats_ready 1 runs only the
 * normalisation (0 is mle_norm_fwd).  Contiguous groups (LayerNorm,
 * GroupNorm, InstanceNorm). */
int mle_norm_fwd_ex(mle_stream stream, const float* x, float* y, float* stats, int batch, int channels, size_t hw,
                    int groups, float eps, void* ws, size_t ws_bytes, int stats_ready);
/* y = a + b[i mod b_period] (the residual Add, b_period = the size; MatPE's
 * table add, b_period = rows * cols) fused with the first pass of the group
 * normalisation that reads y: the per-chunk statistics go to that
 * normalisation's workspace, computed exactly as mle_norm_fwd computes them
 * from y, so the normalised output is bit-identical.  (Add forward,
 * Engine/engine.cu:1630-1672; MatPE, Engine/kernels.cu:166; LayerMean and
 * LayerStd, Engine/kernels.cu:541, 670.) */
/* A group normalisation followed by an activation (GroupNorm -> SiLU in the
 * residual block, Engine/diffusion.cu:129-137; SILU / RELU / GELU ops,
 * Engine/engine.cu:2650-2780):
 *   mle_norm_fwd_act: mle_norm_fwd_ex, and act_out = act(y) from the same pass.
 *   mle_norm_bwd_act: dy (+)= act'(y) * da (accumulate_dy 1 adds), stored --
 *     the activation's backward -- then mle_norm_bwd from that dy, with its
 *     statistics pass reading da and y once for both.
 * The same values as the activation and normalisation kernels run one after
 * the other. */
int mle_norm_fwd_act(mle_stream stream, const float* x, float* y, float* act_out, int kind, float* stats, int batch,
                     int channels, size_t hw, int groups, float eps, void* ws, size_t ws_bytes, int stats_ready);
/* GroupNorm -> activation -> Broadcast_Channel in one pass: y = the
 * normalisation (as mle_norm_fwd_ex), out = act(y) + cbias[channel]
 * (GroupNorm, Engine/kernels.cu:818-834; the activation forward,
 * Engine/kernels.cu:1214-1328; broadcast_add, Engine/kernels.cu:1661).  The
 * activation's own output is not written.  hw % 4 == 0. */
int mle_norm_fwd_act_bias(mle_stream stream, const float* x, float* y, float* out, int kind, const float* cbias,
                          float* stats, int batch, int channels, size_t hw, int groups, float eps, void* ws,
                          size_t ws_bytes, int stats_ready);
int mle_norm_bwd_act(mle_stream stream, const float* y, const float* da, int kind, float* dy, int accumulate_dy,
                     float* dx, const float* stats, int batch, int channels, size_t hw, int groups, float eps,
                     int reference_layout, void* ws, size_t ws_bytes, int accumulate);
int mle_add_norm_partials(mle_stream stream, const float* a, const float* b, size_t b_period, float* y, int batch,
                          int channels, size_t hw, int groups, void* ws, size_t ws_bytes);
/* dx (+)= r * (dy - sum(dy)/N - y * sum(dy*y)/N), r = rsqrt(ssd/N + eps).
 * LayerBackward / GroupBackward (Engine/kernels.cu:849-896) after the ggamma
 * reductions of Engine/engine.cu:3116-3130 / 3262-3276.  With
 * reference_layout != 0 and groups == 1 only the first batch*hw elements get
 * a gradient, as LayerBackward's guard does for channels > 1 (the rest are
 * untouched, or 0 when assigning). */
int mle_norm_bwd(mle_stream stream, const float* y, const float* dy, float* dx, const float* stats,
                 int batch, int channels, size_t hw, int groups, float eps, int reference_layout,
                 void* ws, size_t ws_bytes, int accumulate);
/* mle_norm_bwd (or mle_norm_bwd_act) in its two passes, for a normalisation
 * whose input is produced by an Add or MatPE that no other node reads after
 * the normalisation's backward (the pre-norm transformer block,
 * Engine/transformer.cu:647-661):
 *   mle_norm_bwd_partials: the first pass (the sums of dy and dy*y) into ws,
 *     at the normalisation's place in the backward; with kind >= 0 it first
 *     forms dy (+)= act'(y) * da (accumulate_dy), stored, as mle_norm_bwd_act;
 *   mle_norm_bwd_apply_add: the second pass at the producer's place (Add
 *     backward, Engine/engine.cu:1650-1672; MatPE, 1263-1296): dx (+)= the
 *     normalisation's input gradient -- the producer's output gradient --
 *     and the new dx (+)= into dxa and dxb, the producer's input gradients
 *     (each with its own accumulate flag; dxb may be null), in one pass.
 *     With accumulate, dx = dx_in + the normalisation's gradient: dx_in is
 *     dx itself when null, or the producer's other consumers' gradient kept
 *     elsewhere (a pass-through's, read in place of a copy into dx).
 * The same values, bit for bit, as mle_norm_bwd (_act) followed by the
 * producer's gradient copies (mle_accumulate2 / accumulate at scale 1). */
int mle_norm_bwd_partials(mle_stream stream, const float* y, float* dy, const float* da, int kind, int accumulate_dy,
                          int batch, int channels, size_t hw, int groups, int reference_layout, void* ws,
                          size_t ws_bytes);
int mle_norm_bwd_apply_add(mle_stream stream, const float* y, const float* dy, float* dx, int accumulate,
                           const float* dx_in, float* dxa, int accumulate_a, float* dxb, int accumulate_b,
                           const float* stats, int batch, int channels, size_t hw, int groups, float eps,
                           int reference_layout, void* ws, size_t ws_bytes);

/* BatchNorm: per-channel statistics over (batch, H, W), gamma 1, beta 0.
 * stats[2c] = mean, stats[2c+1] = sum (x - mean)^2; y = (x - mean) * r with
 * r = rsqrt(ssd/N + eps), N = batch * hw.  BatchMean / BatchStd / BNorm
 * (Engine/kernels.cu:574-604, 701-730, 806-816) as composed by
 * GraphOperations::BatchNorm (Engine/engine.cu:3148-3210). */
size_t mle_batchnorm_ws_bytes(int batch, int channels, size_t hw);
int mle_batchnorm_fwd(mle_stream stream, const float* x, float* y, float* stats,
                      int batch, int channels, size_t hw, float eps, void* ws, size_t ws_bytes);
/* dx (+)= r * (dy - sum(dy)/N - y * sum(dy*y)/N) per channel.  BatchBackward
 * (Engine/kernels.cu:864-876) after the ggamma reductions of
 * Engine/engine.cu:3185-3194; accumulate = 0 assigns. */
int mle_batchnorm_bwd(mle_stream stream, const float* y, const float* dy, float* dx, const float* stats,
                      int batch, int channels, size_t hw, float eps, void* ws, size_t ws_bytes, int accumulate);

/* The reference's RMSNorm: an L2 normalisation y = x / sqrtf(sum x^2) along
 * each row (type 0) or each column (type 1) of every [rows x cols] matrix;
 * norms[] gets one value per line.  SumSquaredSqrtCols / SumSquaredSqrtRows +
 * Scale_arr (Engine/kernels.cu:2246-2277, 2058-2071), GraphOperations::RMSNorm
 * (Engine/engine.cu:2613-2648). */
int mle_rmsnorm_fwd(mle_stream stream, const float* x, float* y, float* norms, int bc, int rows, int cols, int type);
/* dx (+)= (dy - y * <dy, y>) / norm along the same line.
 * Accumulate_rmsnorm_kernel (Engine/kernels.cu:2073-2105). */
int mle_rmsnorm_bwd(mle_stream stream, const float* y, const float* dy, const float* norms, float* dx,
                    int bc, int rows, int cols, int type, int accumulate);

/* ------------------------------------------------------------------------- */
/* Layout (U-Net skip concatenation, transposed-convolution weights)         */
/* ------------------------------------------------------------------------- */

/* y [batch][c1 + c2][h][w]: the first c1 channels are x1 [batch][c1][h1][w1]
 * cropped to its centred h x w window (offsets (h1-h)/2, (w1-w)/2), the rest
 * are x2 [batch][c2][h][w].  CopynCrop + Channel_Concat (Engine/kernels.cu:
 * 1330-1348, 1408-1419) as composed by GraphOperations::CopyCrop
 * (Engine/engine.cu:2855-2920).  h1 < h or w1 < w is rejected
 * (MLE_ERR_UNSUPPORTED): the reference reads outside x1 there. */
int mle_copy_crop_fwd(mle_stream stream, const float* x1, const float* x2, float* y,
                      int batch, int c1, int h1, int w1, int c2, int h, int w);
/* dx1 (+)= dy[:, :c1] at the centred window (outside it: unchanged, or 0 when
 * assigning); dx2 (+)= dy[:, c1:].  Channel_Split + PaddingCrop
 * (Engine/kernels.cu:1421-1433, 1350-1369).  accumulate* = 0 assigns. */
int mle_copy_crop_bwd(mle_stream stream, const float* dy, float* dx1, float* dx2,
                      int batch, int c1, int h1, int w1, int c2, int h, int w, int accumulate1, int accumulate2);
/* dst[i][o][k] (+)= src[o][i][k] for k < khw: swaps the two leading axes of a
 * convolution weight.  Convolute2DT keeps [out][inp][kh][kw] weights
 * (Includes/engine.h:257-280); with them swapped its forward, input gradient
 * and weight gradient (CVT2D / CVT2D_GradInput / GVT2D, Engine/kernels.cu:
 * 1091-1212) are the convolution's dgrad, forward and wgrad below. */
int mle_weight_swap(mle_stream stream, const float* src, float* dst, int o, int i, int khw, int accumulate);

/* ------------------------------------------------------------------------- */
/* Convolution (NCHW input, OIHW weights), implicit GEMM on fp32 MFMA        */
/* ------------------------------------------------------------------------- */

/* y = conv(x, w) + b (b may be NULL).  CV2D (Engine/kernels.cu:985-1019). */
int mle_conv2d_fwd(mle_stream stream, const float* x, const float* w, const float* b, float* y,
                   int n, int cin, int h, int w_in, int cout, int kh, int kw, int pad, int stride);
/* dx (+)= conv_transpose(dy, w).  CV2D_GradInput (Engine/kernels.cu:1053-1089). */
int mle_conv2d_dgrad(mle_stream stream, const float* dy, const float* w, float* dx,
                     int n, int cin, int h, int w_in, int cout, int kh, int kw, int pad, int stride, int accumulate);
size_t mle_conv2d_wgrad_ws_bytes(int n, int cin, int h, int w_in, int cout, int kh, int kw, int pad, int stride);
/* dw = sum_{n,oh,ow} x * dy  (assign).  GV2D (Engine/kernels.cu:1021-1051). */
int mle_conv2d_wgrad(mle_stream stream, const float* x, const float* dy, float* dw,
                     int n, int cin, int h, int w_in, int cout, int kh, int kw, int pad, int stride,
                     void* ws, size_t ws_bytes);
/* mle_conv2d_wgrad, and db[c] (+)= sum_{n,oh,ow} dy[n][c] (db may be NULL;
 * accumulate_db 1 adds, 0 assigns): the bias gradient of Convolute2D's
 * backward (GV2D then Channel_Squeeze1D over dy, Engine/engine.cu:3768-3769)
 * taken from the dy rows the weight-gradient kernel already reads (3x3 pad 1
 * and 1x1 stride 1; other filters run the channel sum after the weight
 * gradient).  Same workspace as mle_conv2d_wgrad. */
int mle_conv2d_wgrad_bias(mle_stream stream, const float* x, const float* dy, float* dw, float* db,
                          int accumulate_db, int n, int cin, int h, int w_in, int cout, int kh, int kw, int pad,
                          int stride, void* ws, size_t ws_bytes);

/* A 3 x 3 (pad 1) and a 1 x 1 (pad 0) convolution of the same input, both
 * stride 1 (ResidualBlock's conv1 and skip convolution, Engine/diffusion.cu:
 * 129-137): the two CV2D forwards (Engine/kernels.cu:985-1019) in one launch,
 * and the two CV2D_GradInput passes (Engine/kernels.cu:1052-1089) adding into
 * the one dx in one launch, dx (+)= dgrad3(dy3) + dgrad1(dy1).  _supported
 * says whether the shapes run on these kernels (otherwise the per-convolution
 * calls do; the paired calls return MLE_ERR_UNSUPPORTED). */
int mle_conv2d_pair_supported(int n, int cin, int h, int w, int cout3, int cout1);
int mle_conv2d_pair_fwd(mle_stream stream, const float* x, int n, int cin, int h, int w, const float* w3,
                        const float* b3, float* y3, int cout3, const float* w1, const float* b1, float* y1, int cout1);
int mle_conv2d_pair_dgrad(mle_stream stream, float* dx, int accumulate, int n, int cin, int h, int w,
                          const float* dy3, const float* w3, int cout3, const float* dy1, const float* w1, int cout1);

/* ------------------------------------------------------------------------- */
/* Optimizer                                                                 */
/* ------------------------------------------------------------------------- */

size_t mle_sqnorm_ws_bytes(size_t n);
/* accum[0] += sum(g^2) in double, deterministic order; nonfinite[0] (if not
 * NULL) is set to 1 when a NaN/Inf gradient is seen.
 * SumSquared + atomicAddDouble (Engine/kernels.cu:1486-1506, 51-63). */
int mle_grad_sqnorm(mle_stream stream, const float* g, size_t n, double* accum, int* nonfinite,
                    void* ws, size_t ws_bytes);
/* s = sqrt(s); s = (s > 1) ? s*scale : scale.  Left unchanged when NaN.
 * Sqrt_Scale type 0 (Engine/kernels.cu:1763-1773). */
int mle_sqrt_scale(mle_stream stream, double* s, double scale);
/* mle_grad_sqnorm, then (sqrt_scale != 0) mle_sqrt_scale(accum, scale) in the
 * launch that finishes the sum: GraphOperations::accumulate's last
 * SumSquared followed by its Sqrt_Scale (Engine/engine.cu:3364-3368). */
int mle_grad_sqnorm_ex(mle_stream stream, const float* g, size_t n, double* accum, int* nonfinite, int sqrt_scale,
                       double scale, void* ws, size_t ws_bytes);
/* One Adam (adamw == 0) or AdamW (adamw != 0) step.  When clip != NULL the
 * gradient is read as g / (float)clip[0] (clipNorm fused into the update).
 * AdamUpdate / AdamWUpdate (Engine/kernels.cu:1508-1534), including the double
 * promotion of (1.0 - b) and powf (Adam) vs pow (AdamW) bias correction. */
int mle_adam_update(mle_stream stream, float* p, const float* g, float* m, float* v, size_t n, int t,
                    float lr, float b1, float b2, float eps, float weight_decay, int adamw,
                    const double* clip);
size_t mle_adamw_clip_ws_bytes(size_t n);
/* Fused global-norm clip + Adam(W) over one flat parameter span (p, g, m, v
 * each contiguous n floats): accumulate -> Sqrt_Scale(scale) -> update with
 * g / s, in three launches and two passes over g (32 bytes per parameter).
 * norm_out (nullable, device double) receives s.  The gradient buffer is not
 * rewritten.  GraphOperations::accumulate + clipNorm + ParameterUpdate
 * (Engine/engine.cu:3362-3384). */
int mle_adamw_clip_fused(mle_stream stream, float* p, const float* g, float* m, float* v, size_t n, int t,
                         float lr, float b1, float b2, float eps, float weight_decay, int adamw,
                         double clip_scale, double* norm_out, void* ws, size_t ws_bytes);
/* No counterpart in the reference.  mle_adamw_clip_fused without a workspace
 * argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc): it calls no
 * allocator.  Its scratch -- s and the per-block norm partials, 65,792 bytes,
 * the largest workspace mle_adamw_clip_fused can ask for -- is a fixed device
 * array, one per GPU, held until the process ends; mle_init looks up its
 * address for the device it makes current (or the first call on another
 * device does).  Every call on a GPU shares that GPU's scratch: calls that
 * overlap on one GPU (two streams or two host threads) race.  Each call writes
 * every scratch value it reads, so nothing carries over from the last call.
 * A span whose workspace would exceed the scratch is rejected with
 * MLE_ERR_UNSUPPORTED (none does: the partial count is capped). */
int mle_adamw_clip_fused_noalloc(mle_stream stream, float* p, const float* g, float* m, float* v, size_t n, int t,
                                 float lr, float b1, float b2, float eps, float weight_decay, int adamw,
                                 double clip_scale, double* norm_out);

/* ------------------------------------------------------------------------- */
/* Integer / index paths (bit-exact)                                         */
/* ------------------------------------------------------------------------- */

/* out[b, s, :] = table[keys[b*max_clen + s], :]; keys < 0 (incl. INT_MIN) give 0.
 * GatherEmbeddings (Engine/kernels.cu:2279-2296). */
int mle_embed_gather(mle_stream stream, float* out, const float* table, const int32_t* keys,
                     int batch, int clen, int max_clen, int dim);
size_t mle_embed_scatter_ws_bytes(int batch, int clen);
/* table[keys[b, s], :] += scale * grad[b, s, :] for keys in [0, vocab),
 * summed per row in token order (deterministic).  With scale = -lr it is
 * KeyUpdate (Engine/kernels.cu:1536-1549) without the race; with scale = 1 and
 * `table` a gradient buffer it is the embedding-table gradient. */
int mle_embed_scatter_add(mle_stream stream, float* table, const float* grad, const int32_t* keys,
                          int batch, int clen, int max_clen, int dim, int vocab, float scale,
                          void* ws, size_t ws_bytes);
/* The embedding-table gradient: dtable[keys[b, s], :] (+)= grad[b, s, :], summed
 * per row in token order; accumulate 0 assigns (dtable is logically zero: rows
 * no token reaches become 0, without a separate fill), 1 adds -- the Embedding
 * backward (KeyUpdate into the table gradient, Engine/kernels.cu:1536-1549). */
int mle_embed_grad(mle_stream stream, float* dtable, const float* grad, const int32_t* keys,
                   int batch, int clen, int max_clen, int dim, int vocab, int accumulate,
                   void* ws, size_t ws_bytes);
/* Bytes of the token index that mle_embed_gather_indexed builds ({start, count,
 * first two tokens} per table row, then the tokens grouped by row in token
 * order); 0 when the vocabulary is above 16384 rows (no index: use
 * mle_embed_gather and mle_embed_grad). */
size_t mle_embed_index_bytes(int batch, int clen, int vocab);
/* mle_embed_gather (keys outside [0, vocab) give zero rows) that, in the same
 * launch, builds the index of the tokens per table row into `index` (16-byte
 * aligned, mle_embed_index_bytes long).  The Embedding forward of a training
 * step: GatherEmbeddings (Engine/kernels.cu:2279-2296). */
int mle_embed_gather_indexed(mle_stream stream, float* out, const float* table, const int32_t* keys,
                             int batch, int clen, int max_clen, int dim, int vocab,
                             void* index, size_t index_bytes);
/* mle_embed_grad for the keys indexed by the last mle_embed_gather_indexed on
 * `index` (same batch, clen and vocab): the same bits, with no key scan --
 * the Embedding backward (KeyUpdate into the table gradient,
 * Engine/kernels.cu:1536-1549). */
int mle_embed_grad_indexed(mle_stream stream, float* dtable, const float* grad, const void* index,
                           int batch, int clen, int dim, int vocab, int accumulate);
/* out[(b*clen + s)*vocab + key] = 1 for valid keys (out must be zeroed).
 * OneHotEmbeddings (Engine/kernels.cu:1551-1560). */
int mle_onehot(mle_stream stream, float* out, const int32_t* keys, int batch, int clen, int max_clen, int vocab);
/* One-hot targets kept up to date across steps: for each token, clear
 * out[token, prev_keys[token]], set out[token, key] and store the key in
 * prev_keys (-1 when invalid).  `out` must be all zero when prev_keys is all -1.
 * Equivalent to fill(0) + OneHotEmbeddings (Engine/transformer.cu:190-196)
 * without rewriting the whole [tokens x vocab] matrix every step. */
int mle_onehot_update(mle_stream stream, float* out, int32_t* prev_keys, const int32_t* keys,
                      int batch, int clen, int max_clen, int vocab);
/* out[r] = first index of the maximum of row r (strict >).  ArgMax (Engine/kernels.cu:2353-2366). */
int mle_argmax(mle_stream stream, const float* x, int rows, int cols, int32_t* out);

/* ------------------------------------------------------------------------- */
/* Launch probe (measurement)                                                */
/* ------------------------------------------------------------------------- */

/* Arm the probe for one kernel family ("gemm_nn", "gemm_nt", "gemm_tn",
 * "gemm_tt", "adam_update", ...) or a comma-separated list of them: every
 * later call of those families records a HIP event pair per kernel it
 * launches, on its own stream, together with its algorithmic flop and byte
 * counts.  NULL or "" disarms.  Host-side bookkeeping only. */
int mle_probe_arm(const char* kernel);
/* Synchronise the recorded events and return totals since arming. */
int mle_probe_read(int* launches, double* total_ms, double* total_flop, double* total_bytes);

/* Device timing: an event recorded on a stream completes when the work
 * queued before it has run; elapsed_ms synchronises `stop` and returns the
 * time between the two.  No reference counterpart (its Timing class reads the
 * host clock, Includes/debugging_utils.h:81-93). */
typedef struct mle_event_s* mle_event;
int mle_event_create(mle_event* ev);
int mle_event_record(mle_event ev, mle_stream stream);
int mle_event_elapsed_ms(mle_event start, mle_event stop, float* ms);
int mle_event_destroy(mle_event ev);

#ifdef __cplusplus
}
#endif
#endif /* MLE_HIP_H */
