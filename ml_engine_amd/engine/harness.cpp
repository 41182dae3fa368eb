// Model harness: builds the benchmark configurations with the GraphOperations
// API and exposes them through a small C interface for the tests and bench.py.
// It drives the engine exactly as a reference application does
// (use_cases/mnist.cu:284-293: zero_grad, forward(calc_loss), backward,
// ParameterUpdate) and adds host access to parameters and gradients.
#include <string.h>

#include <fstream>
#include <unordered_map>

#include <memory>
#include <string>
#include <vector>

#include "engine.h"
#include "mle_models.h"
#include "modules.h"

using mle::check;

namespace {

struct Model {
  int kind = 0;
  GraphOperations go;
  graph root;
  std::vector<AdamParameter*> params;
  std::vector<std::pair<void*, size_t>> inputs;  // device buffers by slot
  std::vector<graph> keep;                       // nodes whose outputs are inputs
  // owned modules
  std::unique_ptr<Linear> l1, l2, ffn1, ffn2, lm;
  std::unique_ptr<MultiHeadAttention> mha;
  std::unique_ptr<Embedding> emb;
  std::unique_ptr<ResidualBlock> rb;
  std::unique_ptr<Convolute2DT> up;
  std::unique_ptr<Convolute2D> conv;
  std::vector<std::unique_ptr<AdamParameter>> loose;  // C2 parameters
  double* clip_scale = nullptr;
  bool adamw = true;
  std::vector<float*> grad_backup;  // mle_model_grads_save
  // mle_model_step_graph: the recorded zero_grad / forward / backward pass
  // (for replay_mode's steps) and whether the last step ran it (the loss is
  // then read from the published value).
  mle_graph replay = nullptr;
  int replay_mode = 0;
  bool loss_in_slot = false;
  // The sequence number the recorded pass publishes its loss with (0: it
  // publishes none, or more than one value), and this model's last loss.
  unsigned replay_seq = 0;
  bool loss_spin = false;  // the slot was cleared before the replay: spin for replay_seq
  float loss = 0.0f;
  graph target;  // C1 / C4: the one-hot target node (mle_model_target_read)
};

void* input_buffer(Model* m, size_t bytes) {
  void* p = mle::alloc_scratch(bytes);
  m->inputs.push_back({p, bytes});
  return p;
}

graph input_node(Model* m, const str& name, int a, int b, int c, int d) {
  auto n = std::make_shared<NodeBackProp>(name, a, b, c, d, 1);
  NodeBackProp* nd = n.get();
  n->lazy_grad_writer = true;  // no backward
  n->zero_grad = [=]() { mle::defer_zero(nd); };
  m->inputs.push_back({n->output, (size_t)n->total * sizeof(float)});
  m->keep.push_back(n);
  return n;
}

void build_c1(Model* m, const long long* d) {
  const int batch = (int)d[0], in = (int)d[1], hid = (int)d[2], cls = (int)d[3];
  auto x = input_node(m, "Input", batch, 1, 1, in);
  auto* labels = static_cast<int32_t*>(input_buffer(m, sizeof(int32_t) * batch));
  m->l1.reset(new Linear(in, hid, "First Linear"));
  m->l2.reset(new Linear(hid, cls, "Projection"));
  auto pred = m->l2->forward(GraphOperations::RELU(m->l1->forward(x)));
  auto target = GraphOperations::OneHot(labels, batch, 1, 1, cls);
  m->target = target;
  m->root = GraphOperations::SoftMaxCrossEntropy(pred, target, true);
  m->params = {&m->l1->W1, &m->l1->B1, &m->l2->W1, &m->l2->B1};
  m->adamw = false;
}

void build_c4(Model* m, const long long* d) {
  const int B = (int)d[0], S = (int)d[1], D = (int)d[2], H = (int)d[3], F = (int)d[4], V = (int)d[5];
  auto* ids = static_cast<int32_t*>(input_buffer(m, sizeof(int32_t) * B * S));
  auto* tgt = static_cast<int32_t*>(input_buffer(m, sizeof(int32_t) * B * S));
  m->emb.reset(new Embedding(V, D, "Token Embedding"));
  m->mha.reset(new MultiHeadAttention(D, D, H, "Block MHA"));
  m->ffn1.reset(new Linear(D, F, "FFN1"));
  m->ffn2.reset(new Linear(F, D, "FFN2"));
  m->lm.reset(new Linear(D, V, "Projection"));
  auto x0 = m->emb->forward(ids, B, S, S);
  auto x = GraphOperations::MatrixPositionalEncoding(x0);
  auto h = GraphOperations::LayerNorm(x);
  auto a = m->mha->forward(h, true);
  auto x2 = GraphOperations::Add(x, a);
  auto f = m->ffn2->forward(GraphOperations::GELU(m->ffn1->forward(GraphOperations::LayerNorm(x2))));
  auto x3 = GraphOperations::Add(x2, f);
  auto logits = m->lm->forward(x3);
  auto target = GraphOperations::OneHot(tgt, B, S, S, V);
  m->target = target;
  m->root = GraphOperations::SoftMaxCrossEntropy(logits, target, true);
  auto& mh = *m->mha;
  m->params = {&m->emb->E, &mh.q.W1, &mh.q.B1, &mh.k.W1, &mh.k.B1, &mh.v.W1, &mh.v.B1, &mh.o.W1, &mh.o.B1,
               &m->ffn1->W1, &m->ffn1->B1, &m->ffn2->W1, &m->ffn2->B1, &m->lm->W1, &m->lm->B1};
}

void build_c5(Model* m, const long long* d) {
  const int N = (int)d[0], Cin = (int)d[1], C = (int)d[2], Hs = (int)d[3], Ws = (int)d[4], groups = (int)d[5],
            tdim = (int)d[6], t = (int)d[7];
  auto x = input_node(m, "Input images", N, Cin, Hs, Ws);
  auto noise = input_node(m, "Noise target", N, C, Hs, Ws);
  m->rb.reset(new ResidualBlock(Cin, C, tdim, 1, groups));
  auto temb = GraphOperations::PositionalEncoding(t, tdim);
  auto out = m->rb->forward(x, temb);
  m->root = GraphOperations::MeanSquaredError(out, noise, true);
  auto& r = *m->rb;
  m->params = {&r.conv1->W1, &r.conv1->B1, &r.conv2->W1, &r.conv2->B1,
               &r.skipconv->W1, &r.skipconv->B1, &r.time_mlp->W1, &r.time_mlp->B1};
}

// U-Net decoder step (Convolute2DT, CopyCrop and the remaining normalisations,
// Engine/engine.cu:2613-3347): a
// transposed convolution upsamples x, CopyCrop concatenates the centred crop
// of a skip tensor in front of it, then BatchNorm, row RMSNorm, InstanceNorm
// and column RMSNorm, with an MSE loss against a target.
// dims {N, Cin, Cout, H, W, Cskip, Hs, Ws, k, stride, pad}
void build_c6(Model* m, const long long* d) {
  const int N = (int)d[0], Cin = (int)d[1], Cout = (int)d[2], H = (int)d[3], W = (int)d[4], Cs = (int)d[5],
            Hs = (int)d[6], Ws = (int)d[7], k = (int)d[8], stride = (int)d[9], pad = (int)d[10];
  const int Ho = (H - 1) * stride - 2 * pad + k, Wo = (W - 1) * stride - 2 * pad + k;
  auto x = input_node(m, "Decoder input", N, Cin, H, W);
  auto skip = input_node(m, "Skip features", N, Cs, Hs, Ws);
  auto target = input_node(m, "Target", N, Cs + Cout, Ho, Wo);
  m->up.reset(new Convolute2DT(Cin, Cout, k, k, stride, pad, "Up"));
  auto h = GraphOperations::CopyCrop(skip, m->up->forward(x));
  h = GraphOperations::RMSNorm(GraphOperations::BatchNorm(h), 0);
  h = GraphOperations::RMSNorm(GraphOperations::InstanceNorm(h), 1);
  m->root = GraphOperations::MeanSquaredError(h, target, true);
  m->params = {&m->up->W1, &m->up->B1};
}

// C2: a flat set of parameters; each parameter is carried by a hook node (as
// Linear's output node carries W1/B1) under one track() root.
void build_c2(Model* m, const long long* d, int nd) {
  const int n = (int)d[0];
  size_t total = 0;
  for (int i = 0; i < n; ++i) total += ((size_t)d[1 + i] + 63) & ~size_t(63);
  mle::param_reserve(total);
  graph_tree holders;
  for (int i = 0; i < n; ++i) {
    m->loose.emplace_back(new AdamParameter("param " + std::to_string(i), 1, 1, 1, (int)d[1 + i]));
    AdamParameter* p = m->loose.back().get();
    auto h = std::make_shared<NodeBackProp>("holder " + std::to_string(i), 1, 1, 1, 1, 0);
    h->params = {p};
    h->zero_grad = [=]() { mle::zero(p->grad, p->total); };
    h->accumulate = [=](double* s) { p->accumulate_grad(s); };
    h->clipnorm = [=](const double* s) { p->gradnorm(s); };
    h->updateParams = [=](const float lr, const bool adamw) { p->update(lr, adamw); };
    holders.push_back(h);
    m->params.push_back(p);
  }
  m->root = GraphOperations::track(holders);
  m->clip_scale = static_cast<double*>(mle::alloc_scratch(256));
  (void)nd;
}

// A 1x1 convolution, LayerNorm over its whole [C, H, W] sample (C > 1, where
// the reference's LayerBackward guard matters) and an MSE loss.
// dims {N, Cin, C, H, W}
void build_c7(Model* m, const long long* d) {
  const int N = (int)d[0], Cin = (int)d[1], C = (int)d[2], Hs = (int)d[3], Ws = (int)d[4];
  auto x = input_node(m, "Input", N, Cin, Hs, Ws);
  auto target = input_node(m, "Target", N, C, Hs, Ws);
  m->conv.reset(new Convolute2D(Cin, C, 1, 1, 1, 0, "Conv"));
  m->root = GraphOperations::MeanSquaredError(GraphOperations::LayerNorm(m->conv->forward(x)), target, true);
  m->params = {&m->conv->W1, &m->conv->B1};
}

}  // namespace

extern "C" {

void mle_model_set_lazy_zero(int on) { mle::set_lazy_zero(on != 0); }

void mle_model_set_fusion(int on) { mle::set_sibling_fusion(on != 0); }

void mle_model_set_quirks(int bmmabt_reference_grad, int broadcast_channel_reference_grad,
                          int layernorm_reference_layout) {
  mle::quirks().bmmabt_reference_grad = bmmabt_reference_grad != 0;
  mle::quirks().broadcast_channel_reference_grad = broadcast_channel_reference_grad != 0;
  mle::quirks().layernorm_reference_layout = layernorm_reference_layout != 0;
}

void mle_model_set_seed(unsigned long long seed) { mle::set_init_seed(seed); }

void* mle_model_create(int kind, const long long* dims, int ndims) {
  auto* m = new Model();
  m->kind = kind;
  switch (kind) {
    case 1: build_c1(m, dims); break;
    case 2: build_c2(m, dims, ndims); break;
    case 4: build_c4(m, dims); break;
    case 5: build_c5(m, dims); break;
    case 6: build_c6(m, dims); break;
    case 7: build_c7(m, dims); break;
    default:
      delete m;
      return nullptr;
  }
  m->go.nodes = topological_sort(m->root);
  mle::sync("model build");
  return m;
}

void mle_model_destroy(void* h) {
  auto* m = static_cast<Model*>(h);
  if (!m) return;
  mle::sync("model destroy");
  check(mle_graph_destroy(m->replay), "model graph destroy");
  m->go.clear_graph();
  delete m;
}

int mle_model_num_params(void* h) { return (int)static_cast<Model*>(h)->params.size(); }

const char* mle_model_param_name(void* h, int i) { return static_cast<Model*>(h)->params[i]->op_name.c_str(); }

long long mle_model_param_numel(void* h, int i) { return static_cast<Model*>(h)->params[i]->total; }

int mle_model_param_t(void* h, int i) { return static_cast<Model*>(h)->params[i]->t; }

int mle_model_param_io(void* h, int i, int which, void* host, int to_device) {
  auto* m = static_cast<Model*>(h);
  if (i < 0 || i >= (int)m->params.size() || which < 0 || which > 3) return MLE_ERR_INVALID;
  AdamParameter* p = m->params[i];
  float* dev = which == 0 ? p->output : which == 1 ? p->grad : which == 2 ? p->m : p->v;
  const size_t bytes = (size_t)p->total * sizeof(float);
  if (which == 1) {
    if (to_device) {  // overwritten whole
      mle::clip_drop(p);
      p->grad_pending_zero = false;
    } else {
      mle::materialize(p);  // reads the clipped value, as the reference's buffer holds it
    }
  }
  return to_device ? mle_memcpy_h2d(dev, host, bytes, mle::stream()) : mle_memcpy_d2h(host, dev, bytes, mle::stream());
}

// Keep a device copy of every parameter gradient (save) and write it back
// (restore), so a benchmark can start each optimizer step from the same
// gradients without a host round trip.
int mle_model_grads_save(void* h) {
  auto* m = static_cast<Model*>(h);
  if (m->grad_backup.empty()) {
    for (AdamParameter* p : m->params)
      m->grad_backup.push_back(static_cast<float*>(mle::alloc_scratch((size_t)p->total * sizeof(float))));
  }
  for (size_t i = 0; i < m->params.size(); ++i) {
    AdamParameter* p = m->params[i];
    mle::materialize(p);
    int rc = mle_memcpy_d2d(m->grad_backup[i], p->grad, (size_t)p->total * sizeof(float), mle::stream());
    if (rc) return rc;
  }
  return MLE_OK;
}

int mle_model_grads_restore(void* h) {
  auto* m = static_cast<Model*>(h);
  if (m->grad_backup.size() != m->params.size()) return MLE_ERR_INVALID;
  for (size_t i = 0; i < m->params.size(); ++i) {
    AdamParameter* p = m->params[i];
    mle::clip_drop(p);
    p->grad_pending_zero = false;
    int rc = mle_memcpy_d2d(p->grad, m->grad_backup[i], (size_t)p->total * sizeof(float), mle::stream());
    if (rc) return rc;
  }
  return MLE_OK;
}

int mle_model_input(void* h, int slot, const void* host, size_t bytes) {
  auto* m = static_cast<Model*>(h);
  if (slot < 0 || slot >= (int)m->inputs.size() || bytes > m->inputs[slot].second) return MLE_ERR_INVALID;
  return mle_memcpy_h2d(m->inputs[slot].first, host, bytes, mle::stream());
}

int mle_model_step(void* h, float lr, int mode, float clip) {
  auto* m = static_cast<Model*>(h);
  if (m->kind == 2) {
    if (mode & MLE_STEP_ZERO) m->go.zero_grad();
    if (clip > 0.0f) {
      check(mle_fill(mle::stream(), reinterpret_cast<float*>(m->clip_scale), 0.0f, 2), "clip scale reset");
      m->go.accumulate(m->clip_scale);
      m->go.clipNorm(m->clip_scale);
      // the caller reuses its scale buffer before the update (clipNorm must have kept s)
      if (mode & MLE_STEP_CLOBBER_SCALE)
        check(mle_fill(mle::stream(), reinterpret_cast<float*>(m->clip_scale), 0.0f, 2), "clip scale clobber");
    }
    if (mode & MLE_STEP_UPDATE) m->go.ParameterUpdate(nullptr, false, lr, true);
    return MLE_OK;
  }
  m->loss_in_slot = false;
  if (mode & MLE_STEP_ZERO) m->go.zero_grad();
  if (mode & MLE_STEP_FORWARD) {
    m->go.forward(nullptr, true);
    m->loss = GraphOperations::loss;  // read back inside forward(calc_loss)
  }
  if (mode & MLE_STEP_BACKWARD) m->go.backward();
  if (mode & MLE_STEP_UPDATE) m->go.ParameterUpdate(nullptr, false, lr, m->adamw);
  return MLE_OK;
}

int mle_model_step_graph(void* h, float lr, int mode) {
  auto* m = static_cast<Model*>(h);
  const int pass = mode & (MLE_STEP_ZERO | MLE_STEP_FORWARD | MLE_STEP_BACKWARD);
  if (m->kind == 2 || pass == 0) return mle_model_step(h, lr, mode, 0.0f);
  mle_stream s = mle::stream();
  if (!m->replay || m->replay_mode != pass) {
    int rc = mle_graph_destroy(m->replay);
    m->replay = nullptr;
    if (rc) return rc;
    // Record the pass once.  Its host side runs now (the lazy-clearing marks
    // and every other host decision end as after one step, and are the same
    // for every step of this mode); its kernels run on each replay.
    // A one-time state change would be recorded and then repeated by every
    // replay: gradient aliases left by the previous pass (each backward pass
    // copies those over at its start) and a pending clip are applied now,
    // outside the recording.
    for (auto& n : m->go.nodes) mle::resolve_alias(n.get());
    mle::clip_apply_all();
    unsigned issued0 = 0, issued1 = 0;
    rc = mle_scalar_state(nullptr, nullptr, &issued0);
    if (rc) return rc;
    rc = mle_graph_capture_begin(s);
    if (rc) return rc;
    if (pass & MLE_STEP_ZERO) m->go.zero_grad();
    if (pass & MLE_STEP_FORWARD) m->go.forward(nullptr, true);
    if (pass & MLE_STEP_BACKWARD) m->go.backward();
    rc = mle_graph_capture_end(s, &m->replay);
    if (rc) return rc;
    rc = mle_scalar_state(nullptr, nullptr, &issued1);
    if (rc) return rc;
    m->replay_mode = pass;
    m->replay_seq = issued1 == issued0 + 1 ? issued1 : 0u;
  }
  // The previous replay's loss has been read (or there was none), so no
  // earlier replay of this graph can still publish: clear the slot, and the
  // loss read waits for this replay's number only as long as the forward takes.
  m->loss_spin = false;
  if ((pass & MLE_STEP_FORWARD) && m->replay_seq && !m->loss_in_slot) {
    int rc = mle_scalar_clear();
    if (rc) return rc;
    m->loss_spin = true;
  }
  int rc = mle_graph_launch(m->replay, s);
  if (rc) return rc;
  m->loss_in_slot = (pass & MLE_STEP_FORWARD) != 0;
  // The update runs from the host each step: its bias corrections follow
  // the parameters' step counters.
  if (mode & MLE_STEP_UPDATE) m->go.ParameterUpdate(nullptr, false, lr, m->adamw);
  return MLE_OK;
}

int mle_model_target_read(void* h, float* host, size_t count) {
  auto* m = static_cast<Model*>(h);
  if (!m->target || !host || count > (size_t)m->target->total) return MLE_ERR_INVALID;
  mle::materialize_output(m->target.get());  // the engine's read path
  return mle_memcpy_d2h(host, m->target->output, count * sizeof(float), mle::stream());
}

// The loss of this model's last forward.  After a replayed pass it is read
// once the stream has drained: from the published slot when the last value
// published there carries this graph's sequence number, otherwise (another
// model or read published since) from the loss node's own output, which the
// pass's finishing kernel wrote.
float mle_model_loss(void* h) {
  auto* m = static_cast<Model*>(h);
  if (m->loss_in_slot) {
    float v = 0.0f;
    if (m->loss_spin && mle_scalar_expect(mle::stream(), m->replay_seq, &v) == MLE_OK) {
      m->loss = v;
      GraphOperations::loss = v;
      m->loss_in_slot = false;
      m->loss_spin = false;
      return m->loss;
    }
    check(mle_stream_sync(mle::stream()), "loss read-back");
    unsigned published = 0;
    check(mle_scalar_state(&v, &published, nullptr), "loss read-back");
    if (m->replay_seq == 0 || published != m->replay_seq)
      check(mle_memcpy_d2h(&v, m->root->output, sizeof(float), mle::stream()), "loss read-back");
    m->loss = v;
    GraphOperations::loss = v;
    m->loss_in_slot = false;
  }
  return m->loss;
}

// Parameters whose gradient is marked for a pending clip, over all models
// (a destroyed parameter leaves the set).
long long mle_model_clip_pending(void) { return (long long)mle::clip_marked_count(); }

int mle_model_sync(void* h) {
  (void)h;
  return mle_stream_sync(mle::stream());
}

void* mle_model_stream(void* h) {
  (void)h;
  return mle::stream();
}

int mle_model_num_nodes(void* h) { return (int)static_cast<Model*>(h)->go.nodes.size(); }

long long mle_model_node_numel(void* h, int i) {
  auto* m = static_cast<Model*>(h);
  if (i < 0 || i >= (int)m->go.nodes.size()) return -1;
  return m->go.nodes[i]->total;
}

// Node i (topological order) read the way ReadValueAt / printGPU read it:
// which 0 = output, 1 = gradient (a clear or aliased gradient is made
// current first).
int mle_model_node_read(void* h, int i, int which, float* host, size_t count) {
  auto* m = static_cast<Model*>(h);
  if (i < 0 || i >= (int)m->go.nodes.size() || !host) return MLE_ERR_INVALID;
  NodeBackProp* n = m->go.nodes[i].get();
  if (count > (size_t)n->total || !(which ? n->grad : n->output)) return MLE_ERR_INVALID;
  if (which) mle::materialize(n);
  else mle::materialize_output(n);
  return mle_memcpy_d2h(host, which ? n->grad : n->output, count * sizeof(float), mle::stream());
}

// Checkpoints: every parameter's AdamParameter record, in the model's
// parameter order (the modules' save order, e.g. Linear: W1 then B1).
int mle_model_save(void* h, const char* path) {
  auto* m = static_cast<Model*>(h);
  std::ofstream f(path, std::ios::binary);
  if (!f.is_open()) return MLE_ERR_INVALID;
  for (AdamParameter* p : m->params) p->save(f);
  return f.good() ? MLE_OK : MLE_ERR_INVALID;
}

int mle_model_load(void* h, const char* path) {
  auto* m = static_cast<Model*>(h);
  std::ifstream f(path, std::ios::binary);
  if (!f.is_open()) return MLE_ERR_INVALID;
  for (AdamParameter* p : m->params) p->load(f);
  return MLE_OK;
}

namespace {
std::unordered_map<str, int> vocab_of(const char* const* words, int n) {
  std::unordered_map<str, int> v;
  for (int i = 0; i < n; ++i)
    if (words[i]) v[words[i]] = i;
  return v;
}
}  // namespace

int mle_model_temb_save(void* h, const char* path, const char* const* words, int n) {
  auto* m = static_cast<Model*>(h);
  if (!m->emb) return MLE_ERR_INVALID;
  m->emb->save(str(path), vocab_of(words, n));
  return MLE_OK;
}

int mle_model_temb_load(void* h, const char* path, int replace, const char* const* words, int n) {
  auto* m = static_cast<Model*>(h);
  if (!m->emb) return MLE_ERR_INVALID;
  if (replace) return m->emb->load_replace(str(path), vocab_of(words, n));
  std::unordered_map<str, int> v;
  return m->emb->load(str(path), v);
}

}  // extern "C"
