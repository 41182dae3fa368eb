// GraphOperations / NodeBackProp / AdamParameter -- the ML_Engine C++ surface
// (Includes/engine.h:33-255), kept source-compatible for the ops on the
// training hot path, with every kernel launch going through the C ABI of
// include/mle_hip.h on one HIP stream.
//
// What changes underneath (the API does not):
//  * Memory: node outputs and gradients come from two chunked device arenas
//    (one for outputs, one for gradients, so a graph's gradients are contiguous
//    and zero_grad merges into a few fills); parameters live in a flat
//    parameter arena whose slabs hold [params | grads | m | v] contiguously, so
//    the optimizer, the global norm and the clip run as one pass over a span.
//  * Dispatch: forward / backward enqueue the nodes' lambdas in topological
//    order on one stream with no host synchronisation, except where the
//    reference reads a value back (loss of a `last` node).
//  * accumulate() and clipNorm() are public (the reference declares them
//    private and never calls them, Includes/engine.h:112-113).
#pragma once
#include <stdint.h>
#include <fstream>
#include <functional>
#include <iostream>
#include <memory>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "mle_hip.h"

using str = std::string;

// Includes/debugging_utils.h:10-14 and Includes/kernels.h:7-8
static constexpr float XAVIER = 6.0f;
static constexpr bool ADAMW = true;
static constexpr float NORM = 1.0f;
static constexpr float LEARNING_RATE = 1e-4f;
static constexpr bool SHOULDNORM = false;
static constexpr int BLOCK_SIZE = 32;
static constexpr int THREADSPERBLOCK = 512;

struct NodeBackProp;
struct AdamParameter;

// Set on the output of GraphOperations::OneHot: the token ids the one-hot
// matrix is built from, so a consumer can read them instead of the matrix.
struct OneHotSource {
  const int32_t* keys;  // device, [batch][max_clen]
  int batch, clen, max_clen, vocab;
};
using graph = std::shared_ptr<NodeBackProp>;
using graph_tree = std::vector<graph>;
using graphFn = std::function<graph(graph)>;

namespace mle {

// The stream every engine kernel is enqueued on (created on first use).
mle_stream stream();
void set_stream(mle_stream s);
// Abort with the library's message, as CheckError / SafeCudaMalloc do
// (Engine/debug.cu:15-25, Includes/debugging_utils.h:98-110).
void check(int rc, const str& what);
void sync(const str& what = "sync");

// Device allocation for node tensors.  Released blocks are reused by later
// allocations of the same size (graphs rebuilt with the same shapes).
float* alloc_output(size_t n);
float* alloc_grad(size_t n);
void release(float* p, size_t n, bool grad);
// Scratch owned by a node (workspaces, statistics).
void* alloc_scratch(size_t bytes);
// Shared GEMM split-K workspace of at least `bytes`.  All engine kernels run
// in order on one stream, so one buffer serves every GEMM; a larger request
// allocates a larger buffer (earlier ones stay valid for their users).
void* gemm_workspace(size_t bytes);

// Zero a gradient range.  Inside a ZeroBatch scope the range is recorded and
// merged with its neighbours instead of launching one fill per node.
void zero(float* p, size_t n);
struct ZeroBatch {
  ZeroBatch();
  ~ZeroBatch();
};

// Lazy gradient clearing for node (non-parameter) gradients.  zero_grad marks
// a node's gradient as logically zero instead of filling it; the first
// backward kernel that writes the whole gradient assigns instead of adding
// (accumulate_flag returns 0 once, then 1), so neither the fill nor the read
// of the destination happens.  Anything that reads a marked gradient, or
// writes only part of it, calls materialize() first, which fills it.
void defer_zero(NodeBackProp* n);
int accumulate_flag(NodeBackProp* n);
// The buffer holding n's gradient: grad_src when aliased, else grad.
const float* grad_of(const NodeBackProp* n);
// Alias `in`'s gradient to `from`'s (see NodeBackProp::grad_src) when the
// rules allow; returns whether it did (else the caller writes as usual).
bool alias_grad(NodeBackProp* in, const NodeBackProp* from);
bool can_alias_grad(const NodeBackProp* in, const NodeBackProp* from);  // alias_grad's test, without the alias
// Copy an aliased gradient into the node's own buffer and drop the alias.
void resolve_alias(NodeBackProp* n);
void materialize(NodeBackProp* n);
// Parameter gradients are cleared the same way.  A backward that writes the
// gradients of `ps` whole in one launch asks params_write_flag for its mode:
// 0 (assign) when every one of them is marked clear (the marks are taken),
// otherwise the marked ones are filled and 1 (add) is returned.  Readers of
// parameter gradients (update, norm, clip) call materialize_params first,
// which fills the marked ones and leaves a pending clip deferred.
int params_write_flag(const std::vector<NodeBackProp*>& ps);
void materialize_params(const std::vector<AdamParameter*>& ps);
// Lazy zeroing of a loss node's (one-float) output: zero_grad marks it, the
// loss forward clears the mark when it writes the value, readers call
// materialize_output first.
void defer_zero_output(NodeBackProp* n);
void materialize_output(NodeBackProp* n);
// Off: defer_zero fills at once (the reference's behaviour; results are the
// same either way).  On by default.
void set_lazy_zero(bool on);

// Global-norm clip over parameter gradients (GraphOperations::clipNorm).  The
// reference divides every parameter gradient by s in place (ScalePtr,
// Engine/engine.cu:3362, 302).  Here clipNorm records a copy of s taken at the
// call and marks the parameters: their gradients then read as g / s without
// being rewritten.  The fused ParameterUpdate reads g / s inside the update
// pass; anything else that reads a marked gradient or adds into it (backward,
// accumulate, a second clipNorm, ReadValueAt, printGPU, the NaN check, host
// copies) divides it in place first, so every observable value is the
// reference's.  zero_grad and a whole-tensor overwrite drop the mark.
void clip_mark(const std::vector<AdamParameter*>& ps, const double* s);
// The snapshot of s when every parameter of `ps` is marked (the fused update
// reads through it); otherwise divides the marked ones in place and returns null.
const double* clip_view(const std::vector<AdamParameter*>& ps);
void clip_apply(NodeBackProp* p);  // divide this parameter's gradient now, if marked
void clip_apply_all();
void clip_drop(NodeBackProp* p);   // its gradient is being overwritten or zeroed
void clip_clear();
size_t clip_marked_count();        // parameters marked now (each removes itself when destroyed)

// Flat parameter arena.  param_reserve(n) announces n floats of parameters that
// should be contiguous: it sizes the next slab (default 64 Mi floats) and, if
// the current slab cannot hold n more, makes the next allocation open it.
struct ParamSlot {
  int slab;
  size_t offset;
};
void param_reserve(size_t floats);
ParamSlot param_alloc(size_t n, float** p, float** g, float** m, float** v);

// Seed for parameter initialisation (the reference seeds from std::random_device).
void set_init_seed(uint64_t seed);

// Reference behaviours that are bugs, reproduced by default for parity:
//  bmmabt_reference_grad: BMMABT's B gradient is bcmmT(A, dZ) written into B's
//    buffer (Engine/engine.cu:2307), not dZ^T A.
//  broadcast_channel_reference_grad: Broadcast_Channel reduces only the first
//    `width` channels of B's gradient (Channel_Squeeze1D<<<b, ...>>>,
//    Engine/engine.cu:1435).
//  layernorm_reference_layout: LayerNorm's backward gives a gradient only to the
//    first batch*rows*cols elements when channels > 1 (LayerBackward's
//    `idx >= batch*row*col` guard, Engine/kernels.cu:849-862); off, every
//    element gets the per-sample formula.
struct Quirks {
  bool bmmabt_reference_grad = true;
  bool broadcast_channel_reference_grad = true;
  bool layernorm_reference_layout = true;
};
Quirks& quirks();

}  // namespace mle

struct NodeBackProp {
  str op_name;
  graph_tree inputs;
  float* output = nullptr;
  float* grad = nullptr;
  int dim[4];
  long long total;
  bool forward_called = false;
  std::function<void()> forward;
  std::function<void()> backward;
  std::function<void()> free;
  std::function<void()> zero_grad;
  std::function<void()> serious_free;
  std::function<void(const float lr, const bool adamw)> updateParams;
  std::function<void(const double*)> clipnorm;
  std::function<void(double*)> accumulate;
  std::function<void(const bool full)> printparams;
  // Parameters whose hooks this node carries (additive: lets GraphOperations
  // fuse the optimizer, norm and clip over the flat parameter arena).
  std::vector<AdamParameter*> params;
  // Lazy clearing state (additive): the gradient is logically zero but not
  // filled; and whether this node's backward honours that for its inputs (the
  // engine's ops do; for any other backward the dispatcher fills its inputs'
  // marked gradients first).
  bool grad_pending_zero = false;
  // The same for the output of a loss node, which zero_grad zeroes
  // (Zerograd("Node", node->output, 1), Engine/engine.cu:2120, 1945) and the
  // loss forward overwrites: it is filled only if read before that.
  bool output_pending_zero = false;
  // A write of the output left until something reads it (materialize_output
  // runs it before every read while it is set; running it on a current
  // output changes nothing): a one-hot target whose consumers all read its
  // ids.
  std::function<void()> output_refresh;
  // Counted by forward over the nodes it runs: consumers of this node, and
  // those among them that read only its ids (key_target == this node).
  int fwd_consumers = 0, fwd_key_readers = 0;
  NodeBackProp* key_target = nullptr;
  bool lazy_grad_writer = false;
  // Non-null when this node's output is a one-hot matrix of `keys` (additive).
  std::shared_ptr<OneHotSource> onehot;
  // Set by Linear::forward (additive): computes this node's output as its
  // forward does and also, per row and 64-column block, the max and sum of
  // exp(output - max) into rowpart (row stride ldp floats).  A following
  // softmax cross-entropy with key targets takes over the node's forward with
  // it and never reads the output again (the hook is cleared then).
  std::function<void(float* rowpart, int64_t ldp)> forward_rowstats;
  // Set by Add and MatrixPositionalEncoding (additive): computes this node's
  // output as its forward does and also the first pass of a group
  // normalisation of it (`groups` groups) into that normalisation's workspace.
  // A following LayerNorm / GroupNorm takes over the node's forward with it
  // and skips its own statistics pass (the hook is cleared then).
  std::function<void(int groups, void* ws, size_t ws_bytes)> forward_normstats;
  // Set by the normalisations (additive): computes this node's output as its
  // forward does and also act(output) into act_out, in the same pass.  An
  // activation node on this output takes over the forward with it.
  std::function<void(int kind, float* act_out)> forward_act;
  // A normalisation's forward_act with a broadcast channel add after the
  // activation: out = act(y) + cbias[channel], the activation's own output
  // not written (mle_norm_fwd_act_bias).
  std::function<void(int kind, float* out, const float* cbias)> forward_act_bias;
  // Set by Add (additive): its forward with the activation after it and the
  // last MSE node on that activation's output, one pass
  // (mle_add_mse_act_fwd_bwd_read): the loss and its read-back and the early
  // gradients of the activation's output (dx) and of the Add's output (dz);
  // neither the Add's output nor the activation's is written (the MSE node,
  // which takes the Add + activation pass over with it, recomputes them when
  // they are read).
  std::function<void(int kind, const float* t, size_t n, float* loss, float* dx, float* dz, void* ws,
                     size_t ws_bytes, float* loss_host)>
      forward_act_mse;
  // Set by a small Linear (additive): its forward together with a
  // cross-entropy against key targets of its output (the loss's row
  // statistics, loss value and read-back, and the early gradient), one launch
  // (mle_linear_xent_keys_small_read).  The loss node takes the Linear's
  // forward over with it.
  std::function<void(const int32_t* keys, int clen, int max_clen, float* stats, int batch, float* loss,
                     float* dlogits, float* loss_host)>
      forward_xent_small;
  // An activation whose output the normalisation before it writes (the
  // activation kind), else -1.
  int fused_act_kind = -1;
  // Gradient alias: when set, this node's gradient is the content of
  // grad_src, a consumer's gradient buffer that nothing writes again before
  // the next zero_grad, and `grad` is stale.  A pass-through backward (Add,
  // Broadcast_Channel) sets it instead of copying its gradient into an input
  // whose grad is clear, whose only consumer it is, and whose backward reads
  // through mle::grad_of (reads_grad_alias).  Anything else that reads or
  // adds into the gradient copies it over first (mle::materialize,
  // mle::accumulate_flag); zero_grad and each backward pass's start drop it.
  const float* grad_src = nullptr;
  bool reads_grad_alias = false;
  // Early gradient: the last loss node's forward wrote this node's whole
  // gradient into `grad` while the gradient is still clear
  // (grad_pending_zero), as its backward would assign it.  The loss's
  // backward commits it (clears the mark, launches nothing); a read, another
  // writer or zero_grad before that drops it, and the gradient reads as the
  // reference's zero until the backward computes it as usual.
  bool grad_early = false;
  // Convolute2D: the parameter half of its backward (dW assigned, db added),
  // so a fused input gradient (mle::fuse_conv_pair) can take the other half.
  std::function<void()> backward_params;
  // Backward hand-off (additive): an activation whose input is this node, and
  // which is this node's only consumer, leaves its gradient here instead of
  // forming this node's gradient; this node's backward forms it (kind, and
  // whether it adds to the stored gradient) in its own first pass.
  const float* act_grad_in = nullptr;
  int act_grad_kind = -1;
  int act_grad_acc = 0;
  bool takes_act_grad = false;  // this node's backward handles act_grad_in
  // Backward hand-off (additive), from the consumer's side: an activation
  // node offers its kind here, with a test that its backward would be the
  // plain elementwise pass; a Linear that is the activation's only consumer
  // then forms the activation's input gradient in its own backward launch
  // (mle_linear_bwd_act) and sets act_bwd_done, and the activation's
  // backward launches nothing.
  int act_bwd_kind = -1;
  std::function<bool()> act_bwd_plain;
  bool act_bwd_done = false;
  // Backward hand-off (additive), the other way round: a normalisation whose
  // input is this node, and which is the last of this node's consumers to
  // run its backward, runs its first pass and leaves the second here; this
  // node's backward (an Add's or MatPE's) calls it with its inputs' gradients
  // and their accumulate flags, so that one pass writes this node's gradient
  // and its inputs' at this node's place (the same order of additions).
  std::function<void(float* da, int acc_a, float* db, int acc_b)> grad_apply;
  bool takes_norm_grad = false;  // this node's backward handles grad_apply
  // Number of nodes reading this node's output in the graph being
  // back-propagated, and how many of them have run their backward so far
  // (both kept by GraphOperations::backward).
  int consumers = 0;
  int consumers_done = 0;

  virtual void update(const float lr = LEARNING_RATE, const bool W = ADAMW) {}
  NodeBackProp(str name, int batch, int d1, int d2, int d3, int allocation);
  virtual ~NodeBackProp() = default;
  void clear();
  void reshape(std::vector<int> new_dims);
  void reshape(int arr[], const int size = 4);

 private:
  bool owns_ = false;
};

// Wait for all enqueued work; print and exit on a launch or runtime error
// (Includes/debugging_utils.h:95, Engine/debug.cu:15-25).
void CheckError(const str& reason);

float ReadValueAt(const graph& X, const int& idx, const bool flag = false);
void WriteValueAt(const graph& X, const float value, const int& idx, const bool flag = false);

struct AdamParameter : public NodeBackProp {
  float *m, *v;
  int t;
  float b1, b2, epsilon;
  int batch_size;
  float group_norm;
  float weight_decay;
  mle::ParamSlot slot;

  AdamParameter(str n, int out, int in, int row, int col, double norm = NORM);
  // Leaves the pending-clip set (mle::clip_mark), which holds parameters by address.
  ~AdamParameter() override;
  void save(std::ofstream& f) const;
  void load(std::ifstream& f);
  void update(const float lr = LEARNING_RATE, const bool W = ADAMW) override;
  void accumulate_grad(double* global_scale);
  void gradnorm(const double* global_scale);
  void operator=(const AdamParameter& other);
};

void Dimension(graph X);
void Dimension(AdamParameter X);
// The AdamParameter overloads take a const reference where the reference takes
// the parameter by value (Includes/engine.h:87-96): every call that compiles
// against the reference compiles here, without copying the parameter.
void Zerograd(const AdamParameter& X);
void Zerograd(graph X);
void isNan(graph X, const int type = 0);
void isNan(const AdamParameter& X, const int type = 0);
void printGPU(const graph X, const int type = 0);
void printGPU(const AdamParameter& X, const int type = 0);
void printHeadGPU(const graph X, const int type = 0);
void printHeadGPU(const AdamParameter& X, const int type = 0);
int ArgMaxToCPU(const graph& input);
graph_tree topological_sort(const graph& root);

class GraphOperations {
 private:
  static bool calculate_loss;

 public:
  graph_tree nodes;

  static double GB;
  static float loss;

  // Public here; the reference declares both private and never calls them.
  void clipNorm(double* global_scale);
  void accumulate(double* global_scale);

  void ParameterUpdate(const graph& X = nullptr, const bool show = false, const float lr = LEARNING_RATE,
                       const bool adamw = ADAMW);
  void forward(const graph& X = nullptr, const bool calc_loss = false, const bool show = false, const bool time = false,
               const bool check_nan = false);
  void backward(const graph& X = nullptr, const bool show = false, const bool time = false,
                const bool check_nan = false);
  void zero_grad(const graph& X = nullptr, const bool show = false);
  void printParams(const graph& X = nullptr, const bool show = false);
  void printNodes(const graph& X = nullptr, const int show = 0);
  void clear_graph(const graph& X = nullptr, const bool show = false);
  void clean_clear_graph(const graph& X = nullptr, const bool show = false);

  static graph Copy(const graph& X);
  static graph track(const graph_tree& X);
  static graph identity(const graph& X);
  static graph like(const graph& X, const str name = "");
  static graph HeadifytoChannel(const graph& X, const int new_channels);
  static graph DeHeadify(const graph& X);
  static graph PositionalEncoding(const int& t, const int d_model);
  static graph MatrixPositionalEncoding(const graph& X, const int start_idx = 0);
  static graph Broadcast_Channel(const graph& A, const graph& B);
  static graph Scale(const graph& input, const float scale, const bool last = false);
  static graph Add(const graph& A, const graph& B, const bool last = false);
  static graph MeanSquaredError(const graph& prediction, const graph& target, const bool last);
  static graph SoftMaxCrossEntropy(const graph& prediction, const graph& target, const bool last);
  static graph BMM(const graph& A, const graph& B);     // m x n * n x p = m x p
  static graph BMMABT(const graph& A, const graph& B);  // m x n * p x n = m x p
  // Multi-head attention products over [batch, 1, seq, heads * dim]
  // projections without head permutes (additive; MultiHeadAttention uses them):
  // HeadScores = Scale(BMMABT(Headify(Q), Headify(K)), scale) -> [batch, heads, m, p];
  // HeadMix = DeHeadify(BMM(P, Headify(V))) -> [batch, 1, m, heads * dim].
  static graph HeadScores(const graph& Q, const graph& K, const int heads, const float scale);
  static graph HeadMix(const graph& P, const graph& V, const int heads);
  // HeadMix(SOFTMASK / SOFTMAX type 1 (HeadScores(Q, K, heads, scale)), V) in
  // one node that stores no scores (mle_attention_fwd / _bwd): head_dim 64,
  // seq a multiple of 64.  Returns nullptr (building nothing) for other shapes.
  static graph HeadAttention(const graph& Q, const graph& K, const graph& V, const int heads, const float scale,
                             const bool causal);
  static graph SOFTMAX(const graph& X, const int type = 0);
  static graph SOFTMASK(const graph& X, const int type = 0);
  static graph RELU(const graph& input);
  static graph SILU(const graph& input);
  static graph TANH(const graph& input);
  static graph GELU(const graph& input);
  static graph SIGMOID(const graph& input);
  static graph LeakyRELU(const graph& input);
  static graph LayerNorm(const graph& X);
  static graph BatchNorm(const graph& X);
  static graph GroupNorm(const graph& X, const int group = 8);
  static graph InstanceNorm(const graph& X);
  static graph RMSNorm(const graph& input, const int type = 0);  // type 0: row-wise, type 1: column-wise
  static graph CopyCrop(const graph& input1, const graph& input2);
  // Token-id inputs (TextualEmbedding::forward key "T", Engine/transformer.cu:190-196).
  static graph OneHot(const int32_t* keys, int batch, int clen, int max_clen, int vocab);
};

inline graph operator+(const graph& A, const graph& B) { return GraphOperations::Add(A, B); }

class Linear {
 private:
  int in, out;
  const bool bias;

 public:
  AdamParameter W1;
  AdamParameter B1;
  str op_name = "Linear Layer";
  Linear(const int input, const int output, const str name = "", const bool bias = true);
  graph forward(const graph& X);
  bool has_bias() const { return bias; }
  int in_features() const { return in; }
  int out_features() const { return out; }
  void save(std::ofstream& f) const;
  void load(std::ifstream& f);
  void operator=(const Linear& other);
};

// Horizontal fusion of Linear layers that read the same input (e.g. the Q, K
// and V projections of attention).  `outs` are the layers' forward nodes.
// When the layers' weights, biases, outputs and output gradients sit at equal
// strides in their arenas, the nodes' lambdas are rewired:
//  * forward: whichever sibling runs first in a pass computes every
//    Y_i = X W_i + b_i in one batched launch; the others do nothing (every
//    sibling must be evaluated in each forward pass, as the attention
//    projections are);
//  * backward: the last sibling to run computes every dW_i, db_i in one
//    batched launch and dX = sum_i dY_i W_i^T in one grouped launch.
// Same values as one GEMM per layer up to summation order.  Returns false
// (and changes nothing) otherwise.
namespace mle {
bool fuse_sibling_linears(const std::vector<graph>& outs, const std::vector<Linear*>& layers);
// Global switch for the graph fusions (on by default): fuse_sibling_linears,
// the Linear -> SoftMaxCrossEntropy row statistics and MultiHeadAttention's
// fused attention node.  Graphs built while it is off keep one GEMM per
// layer, a loss that reads the logits and the stored attention scores.
void set_sibling_fusion(bool on);
bool fusion_enabled();
}  // namespace mle

class Convolute2D {
 public:
  int inp, out, c, d, pad, stride;
  str name;
  AdamParameter W1, B1;
  Convolute2D(int Input, int Output, int C = 3, int D = 3, int stride = 1, int padding = 1, str param = "");
  void save(std::ofstream& f) const;
  void load(std::ifstream& f);
  graph forward(const graph& X);
};

// A 3 x 3 (pad 1) and a 1 x 1 (pad 0) convolution, both stride 1, of the same
// input (a residual block's first convolution and its skip).  `y3` and `y1`
// are their forward nodes.  When the shapes run on the paired kernels the
// nodes' lambdas are rewired:
//  * forward: whichever runs first in a pass computes both outputs in one
//    launch (mle_conv2d_pair_fwd; the same bits as two launches);
//  * backward: each keeps its own weight and bias gradients; the second to
//    run computes the input gradient of both, dx (+)= dgrad3(dY3) +
//    dgrad1(dY1), in one launch (mle_conv2d_pair_dgrad).
// Both nodes must be evaluated in every pass, as the residual block's are.
// Returns false (and changes nothing) otherwise.
namespace mle {
bool fuse_conv_pair(const graph& y3, const Convolute2D& c3, const graph& y1, const Convolute2D& c1);
}  // namespace mle

// Transposed convolution (Includes/engine.h:257-280, Engine/engine.cu:3819-3900):
// W1 [out, inp, c, d], B1 [1, out, 1, 1]; output (H - 1) * stride - 2 pad + c.
// Runs on the convolution kernels with W1's two leading axes swapped: forward
// is the convolution's dgrad, the input gradient its forward and the weight
// gradient its wgrad.  Input and weight gradients are assigned, as the
// reference's CVT2D_GradInput and GVT2D do.
class Convolute2DT {
 public:
  int inp, out, c, d, pad, stride;
  str name;
  AdamParameter W1, B1;
  Convolute2DT(int Input, int Output, int C = 2, int D = 2, int stride = 2, int padding = 0, str param = "");
  void save(std::ofstream& f) const;
  void load(std::ifstream& f);
  graph forward(const graph& X);
};

// Token embedding table as an AdamParameter: GatherEmbeddings forward
// (Engine/transformer.cu:176-205) and a deterministic scatter-add backward into
// the table gradient.  UpdateSGD applies the reference's KeyUpdate step
// (Engine/transformer.cu:236-245) without its race.
class Embedding {
 public:
  int vocab, dim;
  AdamParameter E;
  Embedding(int vocab, int dim, const str name = "Embedding");
  graph forward(const int32_t* keys, int batch, int clen, int max_clen);
  void UpdateSGD(const graph& X, float lr = LEARNING_RATE);
  // AdamParameter checkpoint record of the table (with its Adam moments).
  void save(std::ofstream& f) const;
  void load(std::ifstream& f);
  // TEMB files (TextualEmbedding::save / load / load_replace,
  // Engine/transformer.cu:246-484): [u32 magic "TEMB"][u32 version 1]
  // [i32 dim][i32 n] then n x ([u32 len][word][i32 row]) then rows 0..n-1 of
  // the table.  `vocab` is the tokenizer's word -> row map (the reference's
  // WordSpace).  Errors are printed and the call returns, as the reference's do.
  // load: replaces `vocab` and table rows 0..n-1; returns n, or -1.
  // load_replace: copies each saved row whose word is in `vocab` to that
  // word's row; returns how many rows were replaced, or -1.
  void save(const str& filepath, const std::unordered_map<str, int>& vocab) const;
  int load(const str& filepath, std::unordered_map<str, int>& vocab);
  int load_replace(const str& filepath, const std::unordered_map<str, int>& vocab);

 private:
  const int32_t* keys_ = nullptr;
  int batch_ = 0, clen_ = 0, max_clen_ = 0;
  void* ws_ = nullptr;
  size_t ws_bytes_ = 0;
};
