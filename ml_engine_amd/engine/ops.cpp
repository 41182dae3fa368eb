// GraphOperations op factories on the hot path (Engine/engine.cu:675-3347):
// each builds a node whose forward / backward lambdas enqueue C ABI kernels on
// the engine stream.  Backward hooks accumulate (+=) into their inputs'
// gradients, except where the reference assigns (identity, SoftMaxCrossEntropy).
// A gradient that zero_grad only marked as clear is written by its first
// writer with assign semantics (mle::accumulate_flag), which gives the same
// values as adding into zeros without filling or reading the buffer.
#include "engine.h"

#include <math.h>
#include <stdio.h>

#include <algorithm>
#include <vector>

using mle::check;

namespace {

inline mle_stream S() { return mle::stream(); }

graph make_node(const str& name, int a, int b, int c, int d) {
  auto n = std::make_shared<NodeBackProp>(name, a, b, c, d, 1);
  n->lazy_grad_writer = true;
  GraphOperations::GB += (double)n->total * sizeof(float) / (1ULL << 30);
  return n;
}

void std_hooks(const graph& node) {
  NodeBackProp* nd = node.get();
  node->free = [=]() { nd->clear(); };
  node->zero_grad = [=]() { mle::defer_zero(nd); };
}

// dst (+)= scale * src over n floats; assigns when dst's gradient is clear.
void add_grad(NodeBackProp* dst, const float* src, double scale, size_t n, const str& what) {
  if (mle::accumulate_flag(dst)) check(mle_accumulate(S(), src, dst->grad, scale, n), what);
  else check(mle_scale_assign(S(), src, dst->grad, scale, n), what);
}

// Operand case of BMM-family inputs: (dim0 > 1) + 2*(dim1 > 1) (Engine/engine.cu:2221-2223).
int bcase(const graph& X) { return (X->dim[0] > 1) + 2 * (X->dim[1] > 1); }

// First-write beta for B's gradient in the BMM family.  The grid follows A's
// batch and channel sizes, so when B is larger along one of them some of B's
// blocks receive no gradient: then the clear gradient is filled and added to.
float b_grad_beta(NodeBackProp* b, int batch, int channels) {
  const bool covered = (b->dim[0] == 1 || b->dim[0] == batch) && (b->dim[1] == 1 || b->dim[1] == channels);
  if (covered) return (float)mle::accumulate_flag(b);
  mle::materialize(b);
  return 1.0f;
}

// Element offset of batch item (b, c) for an operand with broadcast code `flag`
// (batch_chan_offset, Engine/kernels.cu:371-385).
long long bc_off(int flag, int b, int c, int C, long long inner) {
  const int hb = flag & 1, hc = (flag >> 1) & 1;
  const long long cs = hc ? C : 1;
  return (hb ? (long long)b * cs : 0) * inner + (hc ? (long long)c : 0) * inner;
}

// Batched GEMM over the batch x channel grid with the reference's broadcast
// codes.  When every operand's offset is linear in the item index and no two
// items share an output, one batched launch covers the grid.  Otherwise the
// items run one launch at a time, in order: with beta == 1 items that share an
// output accumulate into it (the reference's atomicAdd epilogue), with beta == 0
// the last item's product stays (the reference's unordered assignment).
// first_beta (accumulating calls only): beta of the first write into each
// output block -- 0 when the destination gradient is clear.
void grid_gemm(int ta, int tb, int M, int N, int K, const float* A, int64_t lda, int fa, long long asz, const float* B,
               int64_t ldb, int fb, long long bsz, float beta, float* Cc, int64_t ldc, int fc, long long csz,
               int batch, int channels, const str& what, float first_beta = 1.0f) {
  const int z = batch * channels;
  auto stride_of = [&](int flag, long long inner, int64_t& stride) -> bool {
    // offset(b, c) must equal stride * (b*channels + c)
    if (flag == 0) {
      stride = 0;
      return true;
    }
    if (flag == 3) {
      stride = inner;
      return true;
    }
    if (flag == 1 && channels == 1) {
      stride = inner;
      return true;
    }
    if (flag == 2 && batch == 1) {
      stride = inner;
      return true;
    }
    return false;
  };
  int64_t sa = 0, sb = 0, sc = 0;
  const bool lin = stride_of(fa, asz, sa) && stride_of(fb, bsz, sb) && stride_of(fc, csz, sc);
  const bool shared_out = (sc == 0 && z > 1) || !lin;
  const bool accumulating = beta != 0.0f;
  if (!shared_out) {
    check(mle_gemm(S(), ta, tb, M, N, K, 1.0f, A, lda, sa, B, ldb, sb, accumulating ? first_beta : beta, Cc, ldc, sc,
                   z, nullptr),
          what);
    return;
  }
  std::vector<long long> written;
  for (int b = 0; b < batch; ++b)
    for (int c = 0; c < channels; ++c) {
      const long long oa = bc_off(fa, b, c, channels, asz), ob = bc_off(fb, b, c, channels, bsz),
                      oc = bc_off(fc, b, c, channels, csz);
      float bt = beta;
      if (accumulating) {
        const bool first = std::find(written.begin(), written.end(), oc) == written.end();
        if (first) written.push_back(oc);
        bt = first ? first_beta : 1.0f;
      }
      check(mle_gemm(S(), ta, tb, M, N, K, 1.0f, A + oa, lda, 0, B + ob, ldb, 0, bt, Cc + oc, ldc, 0, 1, nullptr),
            what);
    }
}

graph act_node(const graph& input, int kind, const str& name) {
  const int a = input->dim[0], b = input->dim[1], c = input->dim[2], d = input->dim[3];
  auto node = make_node(name, a, b, c, d);
  node->inputs = {input};
  NodeBackProp *nd = node.get(), *x = input.get();
  node->forward = [=]() { check(mle_act_fwd(S(), kind, x->output, nd->output, nd->total), name + " forward"); };
  // After a normalisation: its pass writes this activation's output too, and
  // when this node is the normalisation's only consumer, the normalisation's
  // backward forms its gradient from ours in its first pass.
  bool fused = false;
  if (mle::fusion_enabled() && input->forward_act) {
    auto fa = input->forward_act;
    input->forward = [fa, kind, nd]() { fa(kind, nd->output); };
    input->forward_act = nullptr;  // one takeover per producer
    input->forward_normstats = nullptr;
    input->forward_rowstats = nullptr;
    input->forward_xent_small = nullptr;
    node->forward = []() {};
    node->fused_act_kind = kind;
    fused = true;
  }
  node->reads_grad_alias = true;
  node->act_bwd_kind = kind;
  node->act_bwd_plain = [=]() { return !(fused && x->takes_act_grad && x->consumers == 1); };
  node->backward = [=]() {
    if (nd->act_bwd_done) {  // the Linear after this node formed our input's gradient
      nd->act_bwd_done = false;
      return;
    }
    if (fused && x->takes_act_grad && x->consumers == 1) {
      x->act_grad_in = mle::grad_of(nd);
      x->act_grad_kind = kind;
      x->act_grad_acc = mle::accumulate_flag(x);
      return;
    }
    check(mle_act_bwd(S(), kind, x->output, mle::grad_of(nd), x->grad, nd->total, mle::accumulate_flag(x)),
          "Deriv " + name);
  };
  std_hooks(node);
  return node;
}

graph softmax_node(const graph& X, int type, bool masked, const str& name) {
  const int a = X->dim[0], b = X->dim[1], c = X->dim[2], d = X->dim[3];
  auto node = make_node(name, a, b, c, d);
  node->inputs = {X};
  NodeBackProp *nd = node.get(), *x = X.get();
  const int axis = type == 0 ? 0 : 1;
  node->forward = [=]() {
    check(mle_softmax_fwd(S(), x->output, nd->output, a * b, c, d, axis, masked ? 1 : 0), name + " forward");
  };
  node->backward = [=]() {
    check(mle_softmax_bwd(S(), nd->output, nd->grad, x->grad, a * b, c, d, axis, mle::accumulate_flag(x)),
          "Deriv " + name);
  };
  std_hooks(node);
  return node;
}

graph norm_node(const graph& X, int groups, const str& name) {
  const int a = X->dim[0], b = X->dim[1], c = X->dim[2], d = X->dim[3];
  const float eps = 1e-5f;  // gamma = 1, beta = 0 (Engine/engine.cu:3083, 3223)
  auto node = make_node(name, a, b, c, d);
  node->inputs = {X};
  const size_t hw = (size_t)c * d;
  const size_t ws_bytes = mle_norm_ws_bytes(a, b, hw, groups);
  void* ws = mle::alloc_scratch(ws_bytes);
  float* stats = static_cast<float*>(mle::alloc_scratch(2 * sizeof(float) * a * groups));
  GraphOperations::GB += (double)(2 * a * groups) * sizeof(float) / (1ULL << 30);
  NodeBackProp *nd = node.get(), *x = X.get();
  // LayerBackward's C == 1 guard (applies to groups == 1 only), as built
  const int ref_layout = mle::quirks().layernorm_reference_layout ? 1 : 0;
  // An Add or MatPE producer computes the statistics pass with its output.
  int ready = 0;
  if (mle::fusion_enabled() && X->forward_normstats) {
    auto fs = X->forward_normstats;
    X->forward = [fs, groups, ws, ws_bytes]() { fs(groups, ws, ws_bytes); };
    X->forward_normstats = nullptr;  // one takeover per producer
    X->forward_act = nullptr;
    X->forward_act_mse = nullptr;
    ready = 1;
  }
  node->forward = [=]() {
    check(mle_norm_fwd_ex(S(), x->output, nd->output, stats, a, b, hw, groups, eps, ws, ws_bytes, ready),
          name + " forward");
  };
  node->forward_act = [=](int kind, float* act_out) {
    check(mle_norm_fwd_act(S(), x->output, nd->output, act_out, kind, stats, a, b, hw, groups, eps, ws, ws_bytes,
                           ready),
          name + " forward (with the activation after it)");
  };
  if (hw % 4 == 0)
    node->forward_act_bias = [=](int kind, float* out, const float* cbias) {
      check(mle_norm_fwd_act_bias(S(), x->output, nd->output, out, kind, cbias, stats, a, b, hw, groups, eps, ws,
                                  ws_bytes, ready),
            name + " forward (with the activation and channel add after it)");
    };
  node->takes_act_grad = true;
  node->reads_grad_alias = true;
  node->backward = [=]() {
    // The activation after this node may have left its gradient (see act_node).
    const float* da = nd->act_grad_in;
    nd->act_grad_in = nullptr;
    // Our gradient: written from da when an activation follows, else read
    // (possibly through an alias left by a pass-through consumer).
    if (da) mle::resolve_alias(nd);
    float* g = da ? nd->grad : const_cast<float*>(mle::grad_of(nd));
    // An Add or MatPE producer whose other consumers are all done: our first
    // pass now, the second at the producer's place, writing its gradient and
    // its inputs'.
    if (mle::fusion_enabled() && x->takes_norm_grad && x->consumers_done + 1 == x->consumers) {
      // The producer's gradient so far may be an alias (a pass-through
      // consumer's gradient, see can_alias_grad): the second pass adds to it
      // there and writes the producer's own gradient whole.
      const float* x_in = x->grad_src;
      int acc_x = 1;
      if (x_in) {
        x->grad_src = nullptr;
        x->grad_pending_zero = false;
      } else {
        acc_x = mle::accumulate_flag(x);
      }
      check(mle_norm_bwd_partials(S(), nd->output, g, da, da ? nd->act_grad_kind : -1, nd->act_grad_acc, a, b, hw,
                                  groups, ref_layout, ws, ws_bytes),
            name + " backward (first pass)");
      x->grad_apply = [=](float* da, int acc_a, float* db, int acc_b) {
        check(mle_norm_bwd_apply_add(S(), nd->output, g, x->grad, acc_x, x_in, da, acc_a, db, acc_b, stats, a, b, hw,
                                     groups, eps, ref_layout, ws, ws_bytes),
              name + " backward (second pass, into the producer's inputs)");
      };
      return;
    }
    if (da) {
      check(mle_norm_bwd_act(S(), nd->output, da, nd->act_grad_kind, nd->grad, nd->act_grad_acc, x->grad, stats, a,
                             b, hw, groups, eps, ref_layout, ws, ws_bytes, mle::accumulate_flag(x)),
            name + " backward (with the activation after it)");
      return;
    }
    check(mle_norm_bwd(S(), nd->output, g, x->grad, stats, a, b, hw, groups, eps, ref_layout, ws, ws_bytes,
                       mle::accumulate_flag(x)),
          name + " backward");
  };
  std_hooks(node);
  return node;
}

}  // namespace

// Copy (Engine/engine.cu:675-687)
graph GraphOperations::Copy(const graph& X) {
  auto node = make_node("Copy of " + X->op_name, X->dim[0], X->dim[1], X->dim[2], X->dim[3]);
  node->inputs = {X};
  NodeBackProp *nd = node.get(), *x = X.get();
  node->forward = [=]() { check(mle_scale_write(S(), x->output, nd->output, 1.0f, nd->total), "Copy forward"); };
  node->backward = [=]() { add_grad(x, nd->grad, 1.0, nd->total, "Copy backward"); };
  std_hooks(node);
  return node;
}

// like (Engine/engine.cu:689-700)
graph GraphOperations::like(const graph& X, const str name) {
  auto node = make_node(name, X->dim[0], X->dim[1], X->dim[2], X->dim[3]);
  node->inputs = {X};
  node->forward = []() {};
  node->backward = []() {};
  std_hooks(node);
  return node;
}

// identity (Engine/engine.cu:701-713): backward assigns.
graph GraphOperations::identity(const graph& X) {
  auto node = make_node(X->op_name, X->dim[0], X->dim[1], X->dim[2], X->dim[3]);
  node->inputs = {X};
  NodeBackProp *nd = node.get(), *x = X.get();
  node->forward = [=]() { check(mle_scale_write(S(), x->output, nd->output, 1.0f, nd->total), "identity forward"); };
  node->backward = [=]() {
    mle::accumulate_flag(x);  // assigns whole gradient: it is no longer clear
    check(mle_scale_write(S(), nd->grad, x->grad, 1.0f, nd->total), "identity backward");
  };
  std_hooks(node);
  return node;
}

// track (Engine/engine.cu:3349-3360): groups roots without allocating.
graph GraphOperations::track(const graph_tree& X) {
  str name = "Tracking: [";
  for (const auto& p : X) name += (p->op_name + " ");
  name += "]";
  auto node = std::make_shared<NodeBackProp>(name, 1, 1, 1, 1, 0);
  node->inputs = X;
  NodeBackProp* nd = node.get();
  node->free = [=]() { nd->clear(); };
  return node;
}

// HeadifytoChannel (Engine/engine.cu:1144-1164)
graph GraphOperations::HeadifytoChannel(const graph& X, const int heads) {
  if (X->dim[1] != 1 || X->dim[3] % heads != 0) {
    std::cerr << "Headify: channel must be 1 and embed must be divisible by heads\n";
    Dimension(X);
    std::exit(1);
  }
  const int b = X->dim[0], seq = X->dim[2], embed = X->dim[3], hd = embed / heads;
  auto node = make_node("Headified " + X->op_name, b, heads, seq, hd);
  node->inputs = {X};
  NodeBackProp *nd = node.get(), *x = X.get();
  node->forward = [=]() { check(mle_headify(S(), x->output, nd->output, b, heads, seq, hd, 0), "Headify forward"); };
  node->backward = [=]() {
    const int flag = mle::accumulate_flag(x) ? 1 : 2;  // 2: the assigning form of the same permutation
    check(mle_headify(S(), nd->grad, x->grad, b, heads, seq, hd, flag), "Headify backward");
  };
  std_hooks(node);
  return node;
}

// DeHeadify (Engine/engine.cu:1166-1178)
graph GraphOperations::DeHeadify(const graph& X) {
  const int b = X->dim[0], heads = X->dim[1], seq = X->dim[2], hd = X->dim[3];
  auto node = make_node("Deheadified " + X->op_name, b, 1, seq, heads * hd);
  node->inputs = {X};
  NodeBackProp *nd = node.get(), *x = X.get();
  node->forward = [=]() { check(mle_headify(S(), x->output, nd->output, b, heads, seq, hd, 2), "DeHeadify forward"); };
  node->backward = [=]() {
    const int flag = mle::accumulate_flag(x) ? 3 : 0;  // 0: the assigning form of the same permutation
    check(mle_headify(S(), nd->grad, x->grad, b, heads, seq, hd, flag), "DeHeadify backward");
  };
  std_hooks(node);
  return node;
}

// PositionalEncoding (Engine/engine.cu:1244-1261): no backward.
graph GraphOperations::PositionalEncoding(const int& t, const int d_model) {
  auto node = make_node("SinoSuodalPosEncoding", 1, 1, 1, d_model);
  node->inputs = {};
  NodeBackProp* nd = node.get();
  const int tt = t;
  node->forward = [=]() { check(mle_timestep_pe(S(), nd->output, tt, d_model), "PositionalEncoding forward"); };
  std_hooks(node);
  return node;
}

// MatrixPositionalEncoding (Engine/engine.cu:1263-1296)
graph GraphOperations::MatrixPositionalEncoding(const graph& X, const int start_idx) {
  if (X->dim[1] != 1) {
    std::cerr << "MatrixPositionalEncoding expects input with channel dimension of 1\n";
    Dimension(X);
    std::exit(1);
  }
  const int batch = X->dim[0], rows = X->dim[2], cols = X->dim[3];
  auto node = make_node("MatrixSinoSuodalPosEncoding", batch, 1, rows, cols);
  node->inputs = {X};
  NodeBackProp *nd = node.get(), *x = X.get();
  // The encoding depends only on (position, dim): tabulated once here, added
  // to every batch item by the forward.
  float* pe = static_cast<float*>(mle::alloc_scratch((size_t)rows * cols * sizeof(float)));
  check(mle_matpe_table(S(), pe, rows, cols, start_idx), "MatPE table");
  node->forward = [=]() {
    check(mle_add_broadcast(S(), x->output, pe, nd->output, batch, (size_t)rows * cols), "MatPE forward");
  };
  node->forward_normstats = [=](int groups, void* ws, size_t ws_bytes) {
    check(mle_add_norm_partials(S(), x->output, pe, (size_t)rows * cols, nd->output, batch, 1, (size_t)rows * cols,
                                groups, ws, ws_bytes),
          "MatPE forward (with the normalisation statistics)");
  };
  node->takes_norm_grad = true;
  node->reads_grad_alias = true;
  node->backward = [=]() {
    if (nd->grad_apply) {  // the normalisation after this node left its second pass (see norm_node)
      auto apply = std::move(nd->grad_apply);
      nd->grad_apply = nullptr;
      apply(x->grad, mle::accumulate_flag(x), nullptr, 0);
      return;
    }
    add_grad(x, mle::grad_of(nd), 1.0, nd->total, "MatPE backward");
  };
  std_hooks(node);
  return node;
}

// Broadcast_Channel (Engine/engine.cu:1401-1446)
graph GraphOperations::Broadcast_Channel(const graph& A, const graph& B) {
  if (A->dim[1] != B->dim[3] || B->dim[1] != 1 || B->dim[2] != 1) {
    std::cout << "Channel mismatch in broadcast channel \n";
    Dimension(A);
    Dimension(B);
    std::exit(1);
  }
  const int batch = A->dim[0], channels = A->dim[1], a = A->dim[2], b = A->dim[3];
  auto node = make_node("Broadcast Channel", batch, channels, a, b);
  node->inputs = {A, B};
  NodeBackProp *nd = node.get(), *pa = A.get(), *pb = B.get();
  const size_t hw = (size_t)a * b;
  const int nreduce = mle::quirks().broadcast_channel_reference_grad ? b : channels;
  node->forward = [=]() {
    check(mle_broadcast_channel_add(S(), pa->output, pb->output, nd->output, batch, channels, hw),
          "Broadcast Add forward");
  };
  // After a normalisation -> activation pair whose outputs only this node
  // reads: the normalisation's pass is deferred to our forward (the channel
  // vector B may come later in the node order) and writes its own output and
  // ours, act(y) + B[c]; the activation's output is recomputed when read.
  NodeBackProp* nrm = (A->fused_act_kind >= 0 && A->inputs.size() == 1) ? A->inputs[0].get() : nullptr;
  if (mle::fusion_enabled() && nrm && nrm->forward_act_bias && pb->total == channels) {
    auto norm_fwd = nrm->forward;  // the pair's pass (normalisation + activation)
    auto fab = nrm->forward_act_bias;
    nrm->forward_act_bias = nullptr;
    const int kind = A->fused_act_kind;
    auto deferred = std::make_shared<bool>(false);
    nrm->forward = [=]() {
      *deferred = nrm->fwd_consumers == 1 && pa->fwd_consumers == 1;
      if (!*deferred) norm_fwd();
    };
    node->forward = [=]() {
      if (*deferred) {
        *deferred = false;
        fab(kind, nd->output, pb->output);
        return;
      }
      check(mle_broadcast_channel_add(S(), pa->output, pb->output, nd->output, batch, channels, hw),
            "Broadcast Add forward");
    };
    // A read of either output before our forward (a NaN check, a print)
    // runs the pair's pass at once; our forward then adds as usual.
    auto flush = [=]() {
      if (!*deferred) return false;
      *deferred = false;
      norm_fwd();
      return true;
    };
    nrm->output_refresh = [=]() { flush(); };
    pa->output_refresh = [=]() {
      if (!flush())
        check(mle_act_fwd(S(), kind, nrm->output, pa->output, pa->total), "activation output (recomputed for a read)");
    };
  }
  node->reads_grad_alias = true;
  node->backward = [=]() {
    // A's gradient is ours: read in place when A allows it, else written.
    if (!mle::alias_grad(pa, nd)) add_grad(pa, mle::grad_of(nd), 1.0, nd->total, "Broadcast Add backward - A grad");
    // Reduces into (possibly only some of) B's channels; a clear gradient is
    // assigned, the rest of it set to 0 in the same launch.
    check(mle_channel_sum_ex(S(), mle::grad_of(nd), batch, channels, hw, nreduce, pb->grad, (size_t)pb->total,
                             mle::accumulate_flag(pb)),
          "Broadcast Add backward - B grad");
  };
  std_hooks(node);
  return node;
}

// Scale (Engine/engine.cu:2523-2551)
graph GraphOperations::Scale(const graph& input, const float scale, const bool last) {
  const int a = input->dim[0], b = input->dim[1], c = input->dim[2], d = input->dim[3];
  auto node = make_node("Scale", a, b, c, d);
  node->inputs = {input};
  NodeBackProp *nd = node.get(), *x = input.get();
  node->forward = [=]() { check(mle_scale_write(S(), x->output, nd->output, scale, nd->total), "Scale forward"); };
  node->backward = [=]() {
    if (last) check(mle_fill(S(), nd->grad, 1.0f, nd->total), "Scale seed");
    add_grad(x, nd->grad, (double)scale, nd->total, "Deriv Scale");
  };
  std_hooks(node);
  return node;
}

// Add (Engine/engine.cu:1630-1672)
graph GraphOperations::Add(const graph& A, const graph& B, const bool last) {
  for (int i = 0; i < 4; ++i)
    if (A->dim[i] != B->dim[i]) {
      std::cout << "Dimension mismatch in Add \n";
      Dimension(A);
      Dimension(B);
      std::exit(1);
    }
  auto node = make_node("Add", A->dim[0], A->dim[1], A->dim[2], A->dim[3]);
  node->inputs = {A, B};
  NodeBackProp *nd = node.get(), *pa = A.get(), *pb = B.get();
  node->forward = [=]() {
    check(mle_scale_add(S(), pa->output, pb->output, nd->output, 1.0f, nd->total), "Add forward");
    if (last) check(mle_read_scalar(S(), nd->output, &GraphOperations::loss), "Add loss");
  };
  if (!last) {
    const int d0 = A->dim[0], d1 = A->dim[1];
    const size_t d23 = (size_t)A->dim[2] * A->dim[3];
    node->forward_normstats = [=](int groups, void* ws, size_t ws_bytes) {
      check(mle_add_norm_partials(S(), pa->output, pb->output, (size_t)nd->total, nd->output, d0, d1, d23, groups, ws,
                                  ws_bytes),
            "Add forward (with the normalisation statistics)");
    };
    node->forward_act = [=](int kind, float* act_out) {
      check(mle_add_act_fwd(S(), pa->output, pb->output, nd->output, act_out, kind, nd->total),
            "Add forward (with the activation after it)");
    };
    node->forward_act_mse = [=](int kind, const float* t, size_t n, float* loss, float* dx, float* dz, void* ws,
                                size_t ws_bytes, float* loss_host) {
      check(mle_add_mse_act_fwd_bwd_read(S(), pa->output, pb->output, nullptr, t, n, kind, loss, dx, dz, ws,
                                         ws_bytes, loss_host),
            "Add forward (with the activation after it and the last MSE)");
    };
    node->takes_act_grad = true;
    node->takes_norm_grad = true;
  }
  node->backward = [=]() {
    if (last) {
      mle::resolve_alias(nd);
      check(mle_fill(S(), nd->grad, 1.0f, nd->total), "Add seed");
    }
    if (nd->grad_apply) {  // the normalisation after this node left its second pass (see norm_node)
      auto apply = std::move(nd->grad_apply);
      nd->grad_apply = nullptr;
      if (pa != pb && pa->grad != pb->grad) {
        const int acc_a = mle::accumulate_flag(pa), acc_b = mle::accumulate_flag(pb);
        apply(pa->grad, acc_a, pb->grad, acc_b);
        return;
      }
      apply(nullptr, 0, nullptr, 0);  // our gradient only; the inputs' below
    }
    if (nd->act_grad_in) {  // the activation after this node left its gradient (see act_node)
      const float* da = nd->act_grad_in;
      nd->act_grad_in = nullptr;
      mle::resolve_alias(nd);  // written below
      if (pa != pb && pa->grad != pb->grad) {
        if (mle::can_alias_grad(pa, nd) && mle::can_alias_grad(pb, nd)) {
          // both inputs read our gradient in place: only ours is written
          check(mle_act_bwd(S(), nd->act_grad_kind, nd->output, da, nd->grad, nd->total, nd->act_grad_acc),
                "Deriv of the activation after Add");
          mle::alias_grad(pa, nd);
          mle::alias_grad(pb, nd);
          return;
        }
        // ours and both input gradients in one pass
        const int acc_a = mle::accumulate_flag(pa), acc_b = mle::accumulate_flag(pb);
        check(mle_act_bwd_add(S(), nd->output, da, nd->act_grad_kind, nd->grad, nd->act_grad_acc, pa->grad, acc_a,
                              pb->grad, acc_b, nd->total),
              "Add backward (with the activation after it)");
        return;
      }
      check(mle_act_bwd(S(), nd->act_grad_kind, nd->output, da, nd->grad, nd->total, nd->act_grad_acc),
            "Deriv of the activation after Add");
    }
    if (pa != pb && pa->grad != pb->grad) {  // one pass over the output gradient
      const bool la = mle::alias_grad(pa, nd), lb = mle::alias_grad(pb, nd);
      const float* g = mle::grad_of(nd);
      if (la && lb) return;
      if (la || lb) {
        add_grad(la ? pb : pa, g, 1.0, nd->total, "Add backward");
        return;
      }
      const int acc_a = mle::accumulate_flag(pa), acc_b = mle::accumulate_flag(pb);
      check(mle_accumulate2(S(), g, pa->grad, acc_a, pb->grad, acc_b, nd->total), "Add backward");
      return;
    }
    add_grad(pa, mle::grad_of(nd), 1.0, nd->total, "Add backward - A grad");
    add_grad(pb, mle::grad_of(nd), 1.0, nd->total, "Add backward - B grad");
  };
  node->reads_grad_alias = true;
  std_hooks(node);
  return node;
}

// MeanSquaredError (Engine/engine.cu:1900-1949).  zero_grad clears the loss.
graph GraphOperations::MeanSquaredError(const graph& prediction, const graph& target, const bool last) {
  for (int i = 0; i < 4; ++i)
    if (prediction->dim[i] != target->dim[i]) {
      std::cout << "Dimension mismatch \n MSE dimensions are: \n";
      Dimension(prediction);
      Dimension(target);
      std::exit(1);
    }
  auto node = std::make_shared<NodeBackProp>("MSE", 1, 1, 1, 1, 1);
  node->lazy_grad_writer = true;
  node->inputs = {prediction, target};
  GB += (double)(prediction->total + target->total + 1) * sizeof(float) / (1ULL << 30);
  NodeBackProp *nd = node.get(), *pr = prediction.get(), *tg = target.get();
  const size_t n = prediction->total;
  const size_t ws_bytes = mle_loss_ws_bytes(n);
  void* ws = mle::alloc_scratch(ws_bytes);
  // The activation input whose gradient the last forward also formed early,
  // when the prediction is an activation's output read by nothing else.
  auto act_in = std::make_shared<NodeBackProp*>(nullptr);
  // After an Add -> activation pair whose outputs only this node reads (the
  // pair's pass written by the Add, see act_node): the pair's pass is
  // deferred to our forward, which forms the loss and both early gradients in
  // one pass over the Add's inputs and t; the Add's output and the
  // activation's are recomputed when read (the same bits: a + b, then the
  // activation of it).
  NodeBackProp* add = (last && pr->fused_act_kind >= 0 && pr->inputs.size() == 1) ? pr->inputs[0].get() : nullptr;
  auto add_deferred = std::make_shared<bool>(false);
  std::function<void()> pair_fwd;
  decltype(NodeBackProp::forward_act_mse) fam;
  if (mle::fusion_enabled() && add && add->forward_act_mse && add->total == pr->total) {
    pair_fwd = add->forward;
    fam = add->forward_act_mse;
    add->forward_act_mse = nullptr;  // one takeover per producer
    const int kind = pr->fused_act_kind;
    add->forward = [=]() {
      *add_deferred = calculate_loss && add->fwd_consumers == 1 && pr->fwd_consumers == 1;
      if (!*add_deferred) pair_fwd();
    };
    // A read of either output before our forward (a NaN check, a print) runs
    // the pair's pass at once; our forward then goes the unfused way.
    auto flush = [=]() {
      if (!*add_deferred) return false;
      *add_deferred = false;
      pair_fwd();
      return true;
    };
    NodeBackProp *ia = add->inputs[0].get(), *ib = add->inputs[1].get();
    auto add_refresh = [=]() {
      if (!flush())
        check(mle_scale_add(S(), ia->output, ib->output, add->output, 1.0f, add->total),
              "Add output (recomputed for a read)");
    };
    add->output_refresh = add_refresh;
    pr->output_refresh = [=]() {
      add_refresh();
      check(mle_act_fwd(S(), kind, add->output, pr->output, pr->total), "activation output (recomputed for a read)");
    };
  }
  node->forward = [=]() {
    *act_in = nullptr;
    if (*add_deferred) {
      *add_deferred = false;
      if (pr->grad_pending_zero && !pr->grad_src && add->grad_pending_zero && !add->grad_src) {
        fam(pr->fused_act_kind, tg->output, n, nd->output, pr->grad, add->grad, ws, ws_bytes,
            &GraphOperations::loss);
        pr->grad_early = true;
        add->grad_early = true;
        *act_in = add;
        nd->output_pending_zero = false;  // written whole
        return;
      }
      pair_fwd();  // the pair's own pass, then the loss as below
    }
    if (calculate_loss || !last) {
      NodeBackProp* ai = nullptr;
      if (last && mle::fusion_enabled() && pr->act_bwd_kind >= 0 && pr->fwd_consumers == 1 &&
          pr->inputs.size() == 1 && pr->grad_pending_zero && !pr->grad_src) {
        NodeBackProp* c = pr->inputs[0].get();
        if (c && c->fwd_consumers == 1 && c->total == pr->total && c->grad_pending_zero && !c->grad_src) ai = c;
      }
      if (ai) {
        // The loss, its read-back, the prediction's gradient and the
        // activation input's (the activation's backward) from one pass over
        // that input and t, both held early and committed by our backward.
        check(mle_mse_act_fwd_bwd_read(S(), ai->output, tg->output, n, pr->act_bwd_kind, nd->output, pr->grad,
                                       ai->grad, ws, ws_bytes, &GraphOperations::loss),
              "Scalar MSE (with its gradient and the activation's) in MSE forward");
        pr->grad_early = true;
        ai->grad_early = true;
        *act_in = ai;
      } else if (last && mle::fusion_enabled() && pr->grad_pending_zero && !pr->grad_src) {
        // The loss, its read-back and the prediction's gradient from one pass
        // over x and t: the gradient is held early (NodeBackProp::grad_early)
        // and committed by our backward.
        check(mle_mse_fwd_bwd_read(S(), pr->output, tg->output, n, nd->output, pr->grad, ws, ws_bytes,
                                   &GraphOperations::loss),
              "Scalar MSE (with its gradient) in MSE forward");
        pr->grad_early = true;
      } else if (last) {  // the loss and its read-back in one launch
        check(mle_mse_fwd_read(S(), pr->output, tg->output, n, nd->output, ws, ws_bytes, &GraphOperations::loss),
              "Scalar MSE in MSE forward");
      } else {
        check(mle_mse_fwd(S(), pr->output, tg->output, n, nd->output, ws, ws_bytes), "Scalar MSE in MSE forward");
      }
      nd->output_pending_zero = false;  // written whole
    }
  };
  node->backward = [=]() {
    NodeBackProp* ai = *act_in;
    *act_in = nullptr;
    if (last && pr->grad_early && pr->grad_pending_zero) {  // written by our forward: commit it
      pr->grad_early = false;
      pr->grad_pending_zero = false;
      if (ai && ai->grad_early && ai->grad_pending_zero) {  // and the activation's input gradient
        ai->grad_early = false;
        ai->grad_pending_zero = false;
        pr->act_bwd_done = true;  // the activation's backward has nothing left to form
      }
      return;
    }
    // The prediction may be an activation output our forward did not write
    // (the Add + activation pass taken over above): recomputed before it is read.
    if (pr->output_refresh) mle::materialize_output(pr);
    check(mle_mse_bwd(S(), pr->output, tg->output, last ? nullptr : nd->grad, pr->grad, n, mle::accumulate_flag(pr)),
          "deriv MSE");
  };
  node->free = [=]() { nd->clear(); };
  node->zero_grad = [=]() { mle::defer_zero_output(nd); };
  return node;
}

// SoftMaxCrossEntropy (Engine/engine.cu:2064-2124).  The softmax buffer holds
// the whole prediction (the reference allocates node->total == 1 float for it,
// Engine/engine.cu:2080, and writes past it).  Backward assigns.  When the
// target is a OneHot node, the loss and gradient read its ids instead of the
// dense matrix and the backward recomputes the probabilities from per-row
// (max, sum): the same values with a third of the memory traffic.
graph GraphOperations::SoftMaxCrossEntropy(const graph& prediction, const graph& target, const bool last) {
  for (int i = 0; i < 4; ++i)
    if (prediction->dim[i] != target->dim[i]) {
      std::cout << "Dimension mismatch \n CrossEntropy dimensions are: \n";
      Dimension(prediction);
      Dimension(target);
      std::exit(1);
    }
  const int batch = target->dim[0], channels = target->dim[1], c = target->dim[2], d = target->dim[3];
  auto node = std::make_shared<NodeBackProp>("SoftMaxCrossEntropy Loss", 1, 1, 1, 1, 1);
  node->lazy_grad_writer = true;
  node->inputs = {prediction, target};
  GB += (double)(target->total + 1) * sizeof(float) / (1ULL << 30);
  const size_t n = prediction->total;
  const int rows = batch * channels * c;
  const std::shared_ptr<OneHotSource> oh = target->onehot;
  const bool by_keys = oh && channels == 1 && oh->batch == batch && oh->clen == c && oh->vocab == d;
  if (by_keys) node->key_target = target.get();  // reads the ids, never the matrix
  float* probs = by_keys ? nullptr : mle::alloc_output(n);
  float* stats = by_keys ? mle::alloc_output(2 * (size_t)rows) : nullptr;
  const size_t ws_bytes = mle_loss_ws_bytes(n);
  void* ws = mle::alloc_scratch(ws_bytes);
  NodeBackProp *nd = node.get(), *pr = prediction.get(), *tg = target.get();
  // A Linear prediction writes the row statistics with its output (GEMM
  // epilogue), so the loss never reads the logits back.
  const int64_t ldp = 2 * (int64_t)((d + 63) / 64);
  // Small logits (a classifier head): statistics, loss, read-back and the
  // gradient in one launch; the gradient is held early (grad_early) until our
  // backward commits it.
  const bool small = by_keys && last && mle::fusion_enabled() && rows <= 1024 && d <= 64;
  // A small Linear prediction (a classifier head): its forward and all of the
  // above in one launch, at the Linear's place (its forward is taken over,
  // while it is still its own: the row-statistics hook marks that).
  bool head = false;
  if (small && prediction->forward_xent_small && prediction->forward_rowstats &&
      prediction->total == (long long)rows * d) {
    auto fx = prediction->forward_xent_small;
    auto plain = prediction->forward;
    prediction->forward = [=]() {
      if (!calculate_loss) {  // no loss asked: the Linear alone
        plain();
        return;
      }
      const bool early = pr->grad_pending_zero && !pr->grad_src;
      fx(oh->keys, oh->clen, oh->max_clen, stats, batch, nd->output, early ? pr->grad : nullptr,
         &GraphOperations::loss);
      pr->grad_early = early;
      nd->output_pending_zero = false;
    };
    prediction->forward_xent_small = nullptr;
    prediction->forward_rowstats = nullptr;
    prediction->forward_act = nullptr;
    head = true;
  }
  float* rowpart = nullptr;
  if (!small && by_keys && mle::fusion_enabled() && prediction->forward_rowstats &&
      prediction->total == (long long)rows * d) {
    rowpart = mle::alloc_output((size_t)rows * ldp);
    auto fr = prediction->forward_rowstats;
    prediction->forward = [fr, rowpart, ldp]() { fr(rowpart, ldp); };
    prediction->forward_rowstats = nullptr;
  }
  node->forward = [=]() {
    if (calculate_loss || !last) {
      if (head) return;  // the Linear's forward did it all
      if (small) {
        const bool early = pr->grad_pending_zero && !pr->grad_src;
        check(mle_softmax_xent_keys_small_read(S(), pr->output, oh->keys, oh->clen, oh->max_clen, stats, rows, d,
                                               batch, nd->output, early ? pr->grad : nullptr,
                                               &GraphOperations::loss),
              "SoftMaxCrossEntropy");
        pr->grad_early = early;
        nd->output_pending_zero = false;
        return;
      }
      if (rowpart && last) {
        // the loss and its read-back in one launch
        check(mle_softmax_xent_keys_fwd_rowstats_read(S(), pr->output, rowpart, ldp, oh->keys, oh->clen,
                                                      oh->max_clen, stats, rows, d, nd->output, ws, ws_bytes,
                                                      &GraphOperations::loss),
              "SoftMaxCrossEntropy");
        nd->output_pending_zero = false;
        return;
      }
      if (rowpart)
        check(mle_softmax_xent_keys_fwd_rowstats(S(), pr->output, rowpart, ldp, oh->keys, oh->clen, oh->max_clen,
                                                 stats, rows, d, nd->output, ws, ws_bytes),
              "SoftMaxCrossEntropy");
      else if (by_keys)
        check(mle_softmax_xent_keys_fwd(S(), pr->output, oh->keys, oh->clen, oh->max_clen, stats, rows, d, nd->output,
                                        ws, ws_bytes),
              "SoftMaxCrossEntropy");
      else
        check(mle_softmax_xent_fwd(S(), pr->output, tg->output, probs, rows, d, nd->output, ws, ws_bytes),
              "SoftMaxCrossEntropy");
      nd->output_pending_zero = false;  // written whole
      if (last) check(mle_read_scalar(S(), nd->output, &GraphOperations::loss), "CE loss");
    }
  };
  node->backward = [=]() {
    if (small && pr->grad_early && pr->grad_pending_zero) {  // written by our forward: commit it
      pr->grad_early = false;
      pr->grad_pending_zero = false;
      return;
    }
    mle::accumulate_flag(pr);  // the reference assigns the whole gradient
    const float* up = last ? nullptr : nd->grad;
    if (by_keys)
      check(mle_softmax_xent_keys_bwd(S(), pr->output, stats, oh->keys, oh->clen, oh->max_clen, up, pr->grad, rows, d,
                                      batch),
            "derivative of CE in CE backward");
    else
      check(mle_softmax_xent_bwd(S(), probs, tg->output, up, pr->grad, n, batch), "derivative of CE in CE backward");
  };
  node->free = [=]() {
    nd->clear();
    if (probs) mle::release(probs, n, false);
    if (stats) mle::release(stats, 2 * (size_t)rows, false);
    if (rowpart) mle::release(rowpart, (size_t)rows * ldp, false);
  };
  node->zero_grad = [=]() { mle::defer_zero_output(nd); };
  return node;
}

// BMM (Engine/engine.cu:2205-2258): C = A B; dA += dZ B^T; dB += A^T dZ.
graph GraphOperations::BMM(const graph& A, const graph& B) {
  if (A->dim[3] != B->dim[2]) {
    std::cout << "Dimension mismatch in BMM \n";
    Dimension(A);
    Dimension(B);
    std::exit(1);
  }
  const bool bc_ok = ((A->dim[0] == B->dim[0]) || A->dim[0] == 1 || B->dim[0] == 1) &&
                     ((A->dim[1] == B->dim[1]) || A->dim[1] == 1 || B->dim[1] == 1);
  if (!bc_ok) {
    std::cout << "Batch and Channel mismatch in BMM...\n";
    std::exit(1);
  }
  const int fa = bcase(A), fb = bcase(B), fc = fa > fb ? fa : fb;
  // The node takes A's batch and channel sizes, as the reference does.
  const int batch = A->dim[0], channels = A->dim[1], m = A->dim[2], n = A->dim[3], p = B->dim[3];
  auto node = make_node("BMM", batch, channels, m, p);
  node->inputs = {A, B};
  NodeBackProp *nd = node.get(), *pa = A.get(), *pb = B.get();
  const long long asz = (long long)m * n, bsz = (long long)n * p, csz = (long long)m * p;
  node->forward = [=]() {
    grid_gemm(0, 0, m, p, n, pa->output, n, fa, asz, pb->output, p, fb, bsz, 0.0f, nd->output, p, fc, csz, batch,
              channels, "BMM forward");
  };
  node->backward = [=]() {
    grid_gemm(0, 1, m, n, p, nd->grad, p, fc, csz, pb->output, p, fb, bsz, 1.0f, pa->grad, n, fa, asz, batch, channels,
              "BMM dA = dZ B^T", (float)mle::accumulate_flag(pa));
    grid_gemm(1, 0, n, p, m, pa->output, n, fa, asz, nd->grad, p, fc, csz, 1.0f, pb->grad, p, fb, bsz, batch, channels,
              "BMM dB = A^T dZ", b_grad_beta(pb, batch, channels));
  };
  std_hooks(node);
  return node;
}

// BMMABT (Engine/engine.cu:2260-2314): C = A B^T; dA += dZ B.  The reference's
// dB is bcmmT(A, dZ) with dims (n, m, p): C'[n x p] = A^T (dZ viewed as p x m)^T
// written into B's gradient buffer; mle::quirks() selects it (default) or dZ^T A.
graph GraphOperations::BMMABT(const graph& A, const graph& B) {
  if (A->dim[3] != B->dim[3]) {
    std::cout << "Dimension mismatch in BMMABT \n";
    Dimension(A);
    Dimension(B);
    std::exit(1);
  }
  const int fa = bcase(A), fb = bcase(B), fc = fa > fb ? fa : fb;
  const int batch = A->dim[0], channels = A->dim[1], m = A->dim[2], n = A->dim[3], p = B->dim[2];
  auto node = make_node("BMMABT", batch, channels, m, p);
  node->inputs = {A, B};
  NodeBackProp *nd = node.get(), *pa = A.get(), *pb = B.get();
  const long long asz = (long long)m * n, bsz = (long long)p * n, csz = (long long)m * p;
  const bool ref_grad = mle::quirks().bmmabt_reference_grad;
  node->forward = [=]() {
    grid_gemm(0, 1, m, p, n, pa->output, n, fa, asz, pb->output, n, fb, bsz, 0.0f, nd->output, p, fc, csz, batch,
              channels, "BMMABT forward");
  };
  node->backward = [=]() {
    grid_gemm(0, 0, m, n, p, nd->grad, p, fc, csz, pb->output, n, fb, bsz, 1.0f, pa->grad, n, fa, asz, batch, channels,
              "BMMABT dA = dZ B", (float)mle::accumulate_flag(pa));
    if (ref_grad)
      grid_gemm(1, 1, n, p, m, pa->output, n, fa, asz, nd->grad, m, fc, csz, 1.0f, pb->grad, p, fb, bsz, batch,
                channels, "BMMABT dB (reference bcmmT)", b_grad_beta(pb, batch, channels));
    else
      grid_gemm(1, 0, p, n, m, nd->grad, p, fc, csz, pa->output, n, fa, asz, 1.0f, pb->grad, n, fb, bsz, batch,
                channels, "BMMABT dB = dZ^T A", b_grad_beta(pb, batch, channels));
  };
  std_hooks(node);
  return node;
}

// Attention scores per head, scale * Q_h K_h^T, read straight from the
// [batch, 1, seq, heads * dim] projections: HeadifytoChannel(Q), HeadifytoChannel(K),
// BMMABT and Scale of MultiHeadAttention (Engine/transformer.cu:647-654,
// Engine/engine.cu:1144-1164, 2260-2314, 2523-2551) in one node.  The scale is
// the GEMM's alpha (exactly the reference's multiply when it is a power of two).
// Backward: dQ += scale dY K; K's gradient is the reference's bcmmT(Q, dZ) in
// the headified layout (mle::quirks) or the true scale dY^T Q.
graph GraphOperations::HeadScores(const graph& Q, const graph& K, const int heads, const float scale) {
  if (Q->dim[1] != 1 || K->dim[1] != 1 || Q->dim[3] != K->dim[3] || Q->dim[0] != K->dim[0] || Q->dim[3] % heads != 0) {
    std::cerr << "HeadScores: Q and K must be [batch, 1, seq, heads * dim] with the same batch and width\n";
    Dimension(Q);
    Dimension(K);
    std::exit(1);
  }
  const int b = Q->dim[0], m = Q->dim[2], p = K->dim[2], E = Q->dim[3], hd = E / heads;
  auto node = make_node("Head scores", b, heads, m, p);
  node->inputs = {Q, K};
  NodeBackProp *nd = node.get(), *pq = Q.get(), *pk = K.get();
  const bool ref_grad = mle::quirks().bmmabt_reference_grad;
  // The reference's K gradient lands in a headified [b, heads, p, hd] buffer first.
  float* kh = ref_grad ? static_cast<float*>(mle::alloc_scratch(sizeof(float) * (size_t)b * heads * p * hd)) : nullptr;
  const long long qs = (long long)m * E, ks = (long long)p * E, ys = (long long)heads * m * p, yh = (long long)m * p;
  node->forward = [=]() {
    check(mle_gemm_grid(S(), 0, 1, m, p, hd, scale, pq->output, E, qs, hd, pk->output, E, ks, hd, 0.0f, nd->output, p,
                        ys, yh, b, heads, nullptr, 0),
          "HeadScores forward");
  };
  node->backward = [=]() {
    check(mle_gemm_grid(S(), 0, 0, m, hd, p, scale, nd->grad, p, ys, yh, pk->output, E, ks, hd,
                        (float)mle::accumulate_flag(pq), pq->grad, E, qs, hd, b, heads, nullptr, 0),
          "HeadScores dQ = s dY K");
    if (ref_grad) {
      // bcmmT(Q_h, dZ) with dims (hd, m, p): C[hd x p] = Q_h^T (dZ viewed as p x m)^T,
      // written row-major into the head's [p x hd] gradient block.
      check(mle_gemm_grid(S(), 1, 1, hd, p, m, scale, pq->output, E, qs, hd, nd->grad, m, ys, yh, 0.0f, kh, p,
                          (long long)heads * p * hd, (long long)p * hd, b, heads, nullptr, 0),
            "HeadScores dK (reference bcmmT)");
      const int flag = mle::accumulate_flag(pk) ? 1 : 2;
      check(mle_headify(S(), kh, pk->grad, b, heads, p, hd, flag), "HeadScores dK headify backward");
    } else {
      check(mle_gemm_grid(S(), 1, 0, p, hd, m, scale, nd->grad, p, ys, yh, pq->output, E, qs, hd,
                          (float)mle::accumulate_flag(pk), pk->grad, E, ks, hd, b, heads, nullptr, 0),
            "HeadScores dK = s dY^T Q");
    }
  };
  std_hooks(node);
  return node;
}

// Per-head P_h V_h written straight into the [batch, 1, seq, heads * dim]
// concatenation: HeadifytoChannel(V), BMM and DeHeadify of MultiHeadAttention
// (Engine/transformer.cu:655-658, Engine/engine.cu:2205-2258, 1166-1178) in one
// node.  Backward: dP += dO_h V_h^T, dV += P_h^T dO_h.
graph GraphOperations::HeadMix(const graph& P, const graph& V, const int heads) {
  if (V->dim[1] != 1 || P->dim[1] != heads || P->dim[0] != V->dim[0] || P->dim[3] != V->dim[2] ||
      V->dim[3] % heads != 0) {
    std::cerr << "HeadMix: P must be [batch, heads, m, n] and V [batch, 1, n, heads * dim]\n";
    Dimension(P);
    Dimension(V);
    std::exit(1);
  }
  const int b = P->dim[0], m = P->dim[2], n = P->dim[3], E = V->dim[3], hd = E / heads;
  auto node = make_node("Head mix", b, 1, m, E);
  node->inputs = {P, V};
  NodeBackProp *nd = node.get(), *pp = P.get(), *pv = V.get();
  const long long ps = (long long)heads * m * n, ph = (long long)m * n, vs = (long long)n * E, os = (long long)m * E;
  node->forward = [=]() {
    check(mle_gemm_grid(S(), 0, 0, m, hd, n, 1.0f, pp->output, n, ps, ph, pv->output, E, vs, hd, 0.0f, nd->output, E,
                        os, hd, b, heads, nullptr, 0),
          "HeadMix forward");
  };
  node->backward = [=]() {
    check(mle_gemm_grid(S(), 0, 1, m, n, hd, 1.0f, nd->grad, E, os, hd, pv->output, E, vs, hd,
                        (float)mle::accumulate_flag(pp), pp->grad, n, ps, ph, b, heads, nullptr, 0),
          "HeadMix dP = dO V^T");
    check(mle_gemm_grid(S(), 1, 0, n, hd, m, 1.0f, pp->output, n, ps, ph, nd->grad, E, os, hd,
                        (float)mle::accumulate_flag(pv), pv->grad, E, vs, hd, b, heads, nullptr, 0),
          "HeadMix dV = P^T dO");
  };
  std_hooks(node);
  return node;
}

// Fused attention: HeadScores -> SOFTMASK / SOFTMAX (type 1) -> HeadMix of
// MultiHeadAttention (Engine/transformer.cu:647-661) in one node.  The
// forward keeps each key's column statistics in node scratch for the
// backward, which recomputes the score tiles; K's gradient follows
// mle::quirks().bmmabt_reference_grad as HeadScores does.
graph GraphOperations::HeadAttention(const graph& Q, const graph& K, const graph& V, const int heads,
                                     const float scale, const bool causal) {
  if (Q->dim[1] != 1 || K->dim[1] != 1 || V->dim[1] != 1 || Q->dim[0] != K->dim[0] || Q->dim[0] != V->dim[0] ||
      Q->dim[2] != K->dim[2] || Q->dim[2] != V->dim[2] || Q->dim[3] != K->dim[3] || Q->dim[3] != V->dim[3] ||
      heads <= 0 || Q->dim[3] % heads != 0)
    return nullptr;
  const int b = Q->dim[0], seq = Q->dim[2], E = Q->dim[3], hd = E / heads;
  if (hd != 64 || seq % 64 != 0 || (double)b * heads > 65535.0 || (double)b * seq * E * 4.0 >= 2147483647.0)
    return nullptr;
  auto node = make_node("Attention", b, 1, seq, E);
  node->inputs = {Q, K, V};
  NodeBackProp *nd = node.get(), *pq = Q.get(), *pk = K.get(), *pv = V.get();
  const size_t wsb = mle_attention_ws_bytes(b, heads, seq);
  void* ws = mle::alloc_scratch(wsb);
  const bool kref = mle::quirks().bmmabt_reference_grad;
  node->forward = [=]() {
    check(mle_attention_fwd(S(), pq->output, pk->output, pv->output, nd->output, b, heads, seq, hd, E, scale,
                            causal ? 1 : 0, ws, wsb),
          "Attention forward");
  };
  node->backward = [=]() {
    const int aq = mle::accumulate_flag(pq), ak = mle::accumulate_flag(pk), av = mle::accumulate_flag(pv);
    check(mle_attention_bwd(S(), pq->output, pk->output, pv->output, nd->grad, pq->grad, pk->grad, pv->grad, b, heads,
                            seq, hd, E, scale, causal ? 1 : 0, aq, ak, av, kref ? 1 : 0, ws, wsb),
          "Attention backward");
  };
  std_hooks(node);
  return node;
}

graph GraphOperations::SOFTMAX(const graph& X, const int type) { return softmax_node(X, type, false, "Softmax"); }
graph GraphOperations::SOFTMASK(const graph& X, const int type) { return softmax_node(X, type, true, "Softmask"); }
graph GraphOperations::RELU(const graph& input) { return act_node(input, MLE_RELU, "ReLU"); }
graph GraphOperations::SILU(const graph& input) { return act_node(input, MLE_SILU, "SiLU"); }
graph GraphOperations::TANH(const graph& input) { return act_node(input, MLE_TANH, "TANH"); }
graph GraphOperations::GELU(const graph& input) { return act_node(input, MLE_GELU, "GELU"); }
graph GraphOperations::SIGMOID(const graph& input) { return act_node(input, MLE_SIGMOID, "Sigmoid"); }
graph GraphOperations::LeakyRELU(const graph& input) { return act_node(input, MLE_LEAKY_RELU, "LeakyReLU"); }

// LayerNorm (Engine/engine.cu:3080-3146): statistics over C*H*W of each item.
graph GraphOperations::LayerNorm(const graph& X) { return norm_node(X, 1, "LayerNorm"); }

// GroupNorm (Engine/engine.cu:3212-3282)
graph GraphOperations::GroupNorm(const graph& X, const int group) {
  if (X->dim[1] % group != 0) {
    std::cout << "Groups cannot be cleanly split \n";
    Dimension(X);
    std::exit(1);
  }
  return norm_node(X, group, "GroupNorm");
}

// InstanceNorm (Engine/engine.cu:3284-3347): per (batch, channel) statistics
// over H*W -- InstanceMean/InstanceStd/INorm/InstanceBackward are the group
// normalisation with one group per channel.
graph GraphOperations::InstanceNorm(const graph& X) { return norm_node(X, X->dim[1], "InstanceNorm"); }

// BatchNorm (Engine/engine.cu:3148-3210): per-channel statistics over
// (batch, H, W), gamma 1, beta 0, eps 1e-5; no running statistics.
graph GraphOperations::BatchNorm(const graph& X) {
  const int a = X->dim[0], b = X->dim[1], c = X->dim[2], d = X->dim[3];
  const float eps = 1e-5f;
  auto node = make_node("BatchNorm", a, b, c, d);
  node->inputs = {X};
  const size_t hw = (size_t)c * d;
  const size_t ws_bytes = mle_batchnorm_ws_bytes(a, b, hw);
  void* ws = mle::alloc_scratch(ws_bytes);
  float* stats = static_cast<float*>(mle::alloc_scratch(2 * sizeof(float) * b));
  GraphOperations::GB += (double)(2 * b) * sizeof(float) / (1ULL << 30);
  NodeBackProp *nd = node.get(), *x = X.get();
  node->forward = [=]() {
    check(mle_batchnorm_fwd(S(), x->output, nd->output, stats, a, b, hw, eps, ws, ws_bytes), "BatchNorm forward");
  };
  node->backward = [=]() {
    check(mle_batchnorm_bwd(S(), nd->output, nd->grad, x->grad, stats, a, b, hw, eps, ws, ws_bytes,
                            mle::accumulate_flag(x)),
          "BatchNorm backward");
  };
  std_hooks(node);
  return node;
}

// RMSNorm (Engine/engine.cu:2613-2648): y = x / ||x|| along each row (type 0)
// or each column (type 1) of every [H x W] matrix.
graph GraphOperations::RMSNorm(const graph& X, const int type) {
  const int a = X->dim[0], b = X->dim[1], c = X->dim[2], d = X->dim[3];
  auto node = make_node("RMSNorm", a, b, c, d);
  node->inputs = {X};
  const size_t lines = (size_t)a * b * (type == 0 ? c : d);
  float* norms = static_cast<float*>(mle::alloc_scratch(sizeof(float) * lines));
  GraphOperations::GB += (double)lines * sizeof(float) / (1ULL << 30);
  NodeBackProp *nd = node.get(), *x = X.get();
  const int t = type == 0 ? 0 : 1;
  node->forward = [=]() { check(mle_rmsnorm_fwd(S(), x->output, nd->output, norms, a * b, c, d, t), "RMSNorm forward"); };
  node->backward = [=]() {
    check(mle_rmsnorm_bwd(S(), nd->output, nd->grad, norms, x->grad, a * b, c, d, t, mle::accumulate_flag(x)),
          "RMSNorm backward");
  };
  std_hooks(node);
  return node;
}

// CopyCrop (Engine/engine.cu:2855-2920): input1's channels, cropped to
// input2's centred H x W window, followed by input2's channels.
graph GraphOperations::CopyCrop(const graph& input1, const graph& input2) {
  const int batch = input2->dim[0], c2 = input2->dim[1], h = input2->dim[2], w = input2->dim[3];
  const int c1 = input1->dim[1], h1 = input1->dim[2], w1 = input1->dim[3];
  if (input1->dim[0] != batch || h1 < h || w1 < w) {
    std::cout << "CopyCrop needs the same batch and input1 at least as large as input2 \n";
    Dimension(input1);
    Dimension(input2);
    std::exit(1);
  }
  auto node = make_node("CopyNCrop", batch, c1 + c2, h, w);
  node->inputs = {input1, input2};
  NodeBackProp *nd = node.get(), *x1 = input1.get(), *x2 = input2.get();
  node->forward = [=]() {
    check(mle_copy_crop_fwd(S(), x1->output, x2->output, nd->output, batch, c1, h1, w1, c2, h, w),
          "Concatenation in CopynCrop");
  };
  node->backward = [=]() {
    const int acc1 = mle::accumulate_flag(x1), acc2 = mle::accumulate_flag(x2);
    check(mle_copy_crop_bwd(S(), nd->grad, x1->grad, x2->grad, batch, c1, h1, w1, c2, h, w, acc1, acc2),
          "Backward CopynCrop");
  };
  std_hooks(node);
  return node;
}

// One-hot targets from device token ids (TextualEmbedding::forward key "T").
graph GraphOperations::OneHot(const int32_t* keys, int batch, int clen, int max_clen, int vocab) {
  auto node = make_node("OneHot targets", batch, 1, clen, vocab);
  node->inputs = {};
  NodeBackProp* nd = node.get();
  // The matrix is cleared once; each forward then only moves the ones.
  const size_t ntok = (size_t)batch * clen;
  auto* prev = static_cast<int32_t*>(mle::alloc_scratch(ntok * sizeof(int32_t)));
  std::vector<int32_t> none(ntok, -1);
  check(mle_memcpy_h2d(prev, none.data(), ntok * sizeof(int32_t), S()), "OneHot init");
  check(mle_fill(S(), nd->output, 0.0f, nd->total), "OneHot fill");
  auto update = [=]() {
    check(mle_onehot_update(S(), nd->output, prev, keys, batch, clen, max_clen, vocab), "OneHotEmbeddings");
  };
  node->forward = [=]() {
    // Consumers that all read the ids (cross-entropy against key targets)
    // leave the matrix as it is until something reads it; the update then
    // moves the ones from where the last update left them.
    if (nd->fwd_consumers > 0 && nd->fwd_key_readers == nd->fwd_consumers) {
      nd->output_refresh = update;
      return;
    }
    nd->output_refresh = nullptr;
    update();
  };
  node->onehot = std::make_shared<OneHotSource>(OneHotSource{keys, batch, clen, max_clen, vocab});
  std_hooks(node);
  return node;
}
