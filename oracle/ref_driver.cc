// C entry points into the reference's own CPU block reference, for checking
// the oracle restatement against it.
//
// TEST INFRASTRUCTURE ONLY, and built only where the reference tree is
// mounted (oracle/Makefile, target `ref`, output under oracle/_ref/). The
// reference source is compiled where it lies: this translation unit
// includes src/ltx25-block-ref.cc from the reference tree (found through
// -I), which is how the file-local `linear_` (src/ltx25-block-ref.cc:11-28)
// and `stream_ff_` (src/ltx25-block-ref.cc:254-284) become callable here.
// Nothing of the reference is copied into this repository.
#include "ltx25-block-ref.cc"

#include <cstring>
#include <vector>

namespace {

ltx25::Mat make_mat(const float* p, int rows, int cols)
{
  ltx25::Mat m;
  m.rows = rows;
  m.cols = cols;
  m.v.assign(p, p + (std::size_t)rows * cols);
  return m;
}

}  // namespace

extern "C" {

// out[M][N] = x[M][K] . w[N][K]^T + bias[N] through the reference's linear_.
// `bias` may be null.
void ref_linear(const float* x, const float* w, const float* bias, int M,
                int K, int N, float* out)
{
  const ltx25::Mat xm = make_mat(x, M, K);
  const ltx25::Mat wm = make_mat(w, N, K);
  std::vector<float> b;
  if (bias != nullptr) { b.assign(bias, bias + N); }
  ltx25::Mat o;
  ltx25::linear_(xm, wm, b, o);
  std::memcpy(out, o.v.data(), (std::size_t)M * N * sizeof(float));
}

// The reference's public rms_norm (no gain), in place.
void ref_rms_norm(float* x, int rows, int cols, double eps)
{
  ltx25::rms_norm(x, rows, cols, eps);
}

// The reference's feed-forward tail with identity projections and a
// modulation of scale 0, shift 0, gate 1, so that
//   out = x + gelu_tanh(rms_norm(x))
// exactly, every other step being exact. It exposes the GELU that
// stream_ff_ evaluates inline.
void ref_ff_identity(const float* x, int rows, int cols, double eps,
                     float* out)
{
  ltx25::StreamWeights w;
  w.dim = cols;
  w.ff_in.rows = cols;
  w.ff_in.cols = cols;
  w.ff_in.v.assign((std::size_t)cols * cols, 0.0f);
  for (int i = 0; i < cols; ++i) {
    w.ff_in.v[(std::size_t)i * cols + i] = 1.0f;
  }
  w.ff_out = w.ff_in;
  w.scale_shift.assign((std::size_t)9 * cols, 0.0f);
  for (int c = 0; c < cols; ++c) {
    w.scale_shift[(std::size_t)5 * cols + c] = 1.0f;   // gate row
  }
  ltx25::StreamInput s;
  s.x = make_mat(x, rows, cols);
  ltx25::stream_ff_(w, s, eps);
  std::memcpy(out, s.x.v.data(), (std::size_t)rows * cols * sizeof(float));
}

// The reference's attention_ reduced to its per-head gate: q, k and v
// weights zero, v's bias `v_b` [heads * head_dim], the gate logits' weight
// zero and bias `gate_b` [heads], an identity out-projection. Every row's
// softmax then weighs v_b alone, the gate logits are gate_b, and
//   out[r][h * head_dim + d] = v_b[h * head_dim + d] * 2 / (1 + exp(-gate_b[h]))
// as the reference evaluates it (src/ltx25-block-ref.cc:113-125).
void ref_gate_identity(const float* v_b, const float* gate_b, int heads, int head_dim, int rows,
                       float* out)
{
  const int inner = heads * head_dim;
  const int qdim = 8;
  ltx25::AttnWeights w;
  w.heads = heads;
  w.head_dim = head_dim;
  auto zeros = [](int r, int c) {
    ltx25::Mat m;
    m.rows = r;
    m.cols = c;
    m.v.assign((std::size_t)r * c, 0.0f);
    return m;
  };
  w.q_w = zeros(inner, qdim);
  w.k_w = zeros(inner, qdim);
  w.v_w = zeros(inner, qdim);
  w.o_w = zeros(inner, inner);
  for (int i = 0; i < inner; ++i) { w.o_w.v[(std::size_t)i * inner + i] = 1.0f; }
  w.q_b.assign(inner, 0.0f);
  w.k_b.assign(inner, 0.0f);
  w.v_b.assign(v_b, v_b + inner);
  w.o_b.assign(inner, 0.0f);
  w.q_norm.assign(inner, 1.0f);
  w.k_norm.assign(inner, 1.0f);
  w.gate_w = zeros(heads, qdim);
  w.gate_b.assign(gate_b, gate_b + heads);
  const ltx25::Mat x = zeros(rows, qdim);
  const ltx25::Mat ctx = zeros(1, qdim);
  ltx25::Mat o;
  ltx25::attention_(w, x, ctx, nullptr, nullptr, o);
  std::memcpy(out, o.v.data(), (std::size_t)rows * inner * sizeof(float));
}

}  // extern "C"
