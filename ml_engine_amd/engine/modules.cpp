#include "modules.h"

#include <math.h>

// MultiHeadAttention constructor and forward (Engine/transformer.cu:635-661).
MultiHeadAttention::MultiHeadAttention(const int embed_dim_, const int hidden_, const int num_heads_, const str& name_)
    : hidden(hidden_),
      embed_dim(embed_dim_),
      num_heads(num_heads_),
      head_dim(hidden_ / num_heads_),
      name(name_),
      q(embed_dim_, hidden_, name_ + " Query"),
      k(embed_dim_, hidden_, name_ + " Key"),
      v(embed_dim_, hidden_, name_ + " Value"),
      o(hidden_, embed_dim_, name_ + " Output") {
  if (hidden_ % num_heads_ != 0)
    printf("Cannot Split MHA because hidden dim: %i is not divisible by num heads: %i", hidden_, num_heads_);
}

void MultiHeadAttention::save(std::ofstream& f) const {
  q.save(f);
  k.save(f);
  v.save(f);
  o.save(f);
}
void MultiHeadAttention::load(std::ifstream& f) {
  q.load(f);
  k.load(f);
  v.load(f);
  o.load(f);
}

// The reference composes Headify x3, BMMABT, Scale, SOFTMASK, BMM and
// DeHeadify.  With the fusions on and a supported shape, HeadAttention runs
// the whole chain without storing the scores; otherwise HeadScores and
// HeadMix compute the same products on the heads in place (no permuted
// copies, the scale in the GEMM) around the stored softmax.
graph MultiHeadAttention::forward(const graph& X, const bool mask) {
  auto Q = q.forward(X);
  auto K = k.forward(X);
  auto V = v.forward(X);
  // The three projections read X: one launch each way when the arenas allow.
  qkv_fused = mle::fuse_sibling_linears({Q, K, V}, {&q, &k, &v});
  const float scale = 1.0f / sqrtf((float)head_dim);
  graph concat;
  if (mle::fusion_enabled())
    concat = GraphOperations::HeadAttention(Q, K, V, num_heads, scale, mask && Q->dim[2] > 1);
  if (!concat) {
    auto scaled = GraphOperations::HeadScores(Q, K, num_heads, scale);
    auto weights =
        (mask && scaled->dim[2] > 1) ? GraphOperations::SOFTMASK(scaled, 1) : GraphOperations::SOFTMAX(scaled, 1);
    concat = GraphOperations::HeadMix(weights, V, num_heads);
  }
  auto output = o.forward(concat);
  output->op_name = "Multi Head Attention Output";
  return output;
}

// ResidualBlock (Engine/diffusion.cu:109-137).
ResidualBlock::ResidualBlock(const int in_channels, const int out_channels, const int t_hidden, const int stride_,
                             const int groups_)
    : in(in_channels), out(out_channels), hidden(t_hidden), stride(stride_), groups(groups_) {
  conv1.reset(new Convolute2D(in_channels, out_channels, 3, 3, stride_, 1, "ResBlock Conv1"));
  conv2.reset(new Convolute2D(out_channels, out_channels, 3, 3, 1, 1, "ResBlock Conv2"));
  time_mlp.reset(new Linear(t_hidden, out_channels, "ResBlock Time MLP"));
  skipconv.reset(new Convolute2D(in_channels, out_channels, 1, 1, stride_, 0, "ResBlock SkipConv"));
}

void ResidualBlock::save(std::ofstream& f) const {
  conv1->save(f);
  conv2->save(f);
  skipconv->save(f);
  time_mlp->save(f);
}
void ResidualBlock::load(std::ifstream& f) {
  conv1->load(f);
  conv2->load(f);
  skipconv->load(f);
  time_mlp->load(f);
}

graph ResidualBlock::forward(const graph& x, const graph& t_emb) {
  auto c1 = conv1->forward(x);
  auto h = GraphOperations::SILU(GraphOperations::GroupNorm(c1, groups));
  auto time = time_mlp->forward(t_emb);
  h = GraphOperations::Broadcast_Channel(h, time);
  h = GraphOperations::GroupNorm(conv2->forward(h), groups);
  auto skipnet = (in != out || stride != 1) ? skipconv->forward(x) : x;
  // conv1 and the skip convolution read the same x: one launch each way
  if (skipnet != x) mle::fuse_conv_pair(c1, *conv1, skipnet, *skipconv);
  return GraphOperations::SILU(GraphOperations::Add(h, skipnet));
}
