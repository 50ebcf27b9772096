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

}  // extern "C"
