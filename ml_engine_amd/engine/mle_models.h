/* Model harness of libmle_engine.so: builds the benchmark configurations with
 * the GraphOperations API and steps them.  Test and benchmark plumbing, not
 * part of the drop-in boundary (include/mle_hip.h). */
#ifndef MLE_MODELS_H
#define MLE_MODELS_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { MLE_STEP_ZERO = 1, MLE_STEP_FORWARD = 2, MLE_STEP_BACKWARD = 4, MLE_STEP_UPDATE = 8, MLE_STEP_ALL = 15 };
/* kind 2 only: overwrite the clip scale buffer between clipNorm and the update */
enum { MLE_STEP_CLOBBER_SCALE = 16 };

/* kind 1: MLP   dims {batch, in, hidden, classes}            inputs: x f32, labels i32
 * kind 2: flat  dims {n, size_0 .. size_{n-1}}                (accumulate + clip + AdamW)
 * kind 4: block dims {B, S, D, heads, F, V}                   inputs: ids i32, targets i32
 * kind 5: resblock dims {N, Cin, C, H, W, groups, tdim, t}   inputs: x f32, noise f32
 * kind 6: U-Net decoder step dims {N, Cin, Cout, H, W, Cskip, Hs, Ws, k, stride, pad}
 *         (Convolute2DT, CopyCrop, BatchNorm, RMSNorm, InstanceNorm, MSE)
 *                                                             inputs: x, skip, target f32
 * kind 7: 1x1 Convolute2D -> LayerNorm over [C, H, W] -> MSE  dims {N, Cin, C, H, W}
 *                                                             inputs: x, target f32 */
void* mle_model_create(int kind, const long long* dims, int ndims);
void mle_model_destroy(void* h);
/* Reference bugs reproduced (1, default) or fixed (0); see mle::Quirks. */
void mle_model_set_quirks(int bmmabt_reference_grad, int broadcast_channel_reference_grad,
                          int layernorm_reference_layout);
void mle_model_set_seed(unsigned long long seed);
/* 1 (default): zero_grad marks node gradients clear and first writers assign;
 * 0: zero_grad fills them. */
void mle_model_set_lazy_zero(int on);
/* Horizontal fusion of Linear layers that share an input (attention's Q, K, V
 * projections: their input gradient is one grouped sum-of-products GEMM).
 * On by default; applies to models created afterwards. */
void mle_model_set_fusion(int on);
int mle_model_num_params(void* h);
const char* mle_model_param_name(void* h, int i);
long long mle_model_param_numel(void* h, int i);
int mle_model_param_t(void* h, int i);
/* which: 0 params, 1 grads, 2 m, 3 v.  Gradients read as the reference's
 * buffer holds them (a pending clip is applied first); writing one replaces
 * it whole. */
int mle_model_param_io(void* h, int i, int which, void* host, int to_device);
/* Device copy of every parameter gradient, and its write-back (benchmarks
 * that restart each optimizer step from the same gradients). */
int mle_model_grads_save(void* h);
int mle_model_grads_restore(void* h);
int mle_model_input(void* h, int slot, const void* host, size_t bytes);
/* mode: MLE_STEP_* bits; clip > 0 (kind 2) applies accumulate + clipNorm. */
int mle_model_step(void* h, float lr, int mode, float clip);
// The same step with its zero_grad / forward / backward part replayed as one
// recorded graph (recorded on the first call for a mode, recorded again when
// the mode changes) and the update launched from the host.  Same results as
// mle_model_step; mle_model_loss synchronises and reads the published loss.
int mle_model_step_graph(void* h, float lr, int mode);
/* This model's loss from its last forward (eager or replayed). */
float mle_model_loss(void* h);
/* Parameters, over all models, whose gradient awaits a pending clipNorm. */
long long mle_model_clip_pending(void);
// C1 / C4: the first `count` floats of the one-hot target matrix, read the
// way ReadValueAt reads a node output (a matrix left lazy is brought up to
// date first).
int mle_model_target_read(void* h, float* host, size_t count);
int mle_model_sync(void* h);
void* mle_model_stream(void* h);
int mle_model_num_nodes(void* h);
/* Node i of the topological order: its element count, and the first `count`
 * floats of its output (which 0) or gradient (which 1), read the way
 * ReadValueAt reads them. */
long long mle_model_node_numel(void* h, int i);
int mle_model_node_read(void* h, int i, int which, float* host, size_t count);
/* Checkpoint of every parameter (AdamParameter::save records, parameter order). */
int mle_model_save(void* h, const char* path);
int mle_model_load(void* h, const char* path);
/* TEMB file of the block model's embedding table; words[i] is the word of row
 * i (NULL skips).  load: replace = 0 full load (returns the saved vocabulary
 * size), 1 load_replace (returns the rows replaced); -1 on a bad file. */
int mle_model_temb_save(void* h, const char* path, const char* const* words, int n);
int mle_model_temb_load(void* h, const char* path, int replace, const char* const* words, int n);

#ifdef __cplusplus
}
#endif
#endif
