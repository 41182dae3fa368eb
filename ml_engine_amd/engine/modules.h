// Layer compositions used by the benchmark configurations, built only from
// GraphOperations ops: MultiHeadAttention (Includes/transformer.h,
// Engine/transformer.cu:635-661) and the diffusion ResidualBlock
// (Includes/diffusion.h:35-46, Engine/diffusion.cu:109-137).
#pragma once
#include <memory>

#include "engine.h"

class MultiHeadAttention {
 public:
  int hidden, embed_dim, num_heads, head_dim;
  str name;
  Linear q, k, v, o;
  bool qkv_fused = false;  // set by forward: dX of the Q, K, V projections is one grouped GEMM
  MultiHeadAttention(const int embed_dim, const int hidden, const int num_heads, const str& name = "MHA");
  graph forward(const graph& X, const bool mask = true);
  void save(std::ofstream& f) const;
  void load(std::ifstream& f);
};

class ResidualBlock {
 public:
  std::unique_ptr<Convolute2D> conv1, conv2, skipconv;
  std::unique_ptr<Linear> time_mlp;
  int in, out, hidden, stride, groups;
  // `groups` is the GroupNorm group count (the reference always uses the
  // GroupNorm default of 8; the diffusion benchmark block uses 32).
  ResidualBlock(const int in_channels, const int out_channels, const int t_hidden, const int stride = 1,
                const int groups = 8);
  graph forward(const graph& x, const graph& t_emb);
  void save(std::ofstream& f) const;
  void load(std::ifstream& f);
};
