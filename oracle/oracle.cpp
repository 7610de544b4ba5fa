// CPU restatement of the ppocr-rs reference CPU inference path.
//
// TEST INFRASTRUCTURE ONLY.  This file is the parity oracle: it is built into
// liboracle.so and called from tests/, from __graft_entry__.smoke() and from
// bench.py's cpu_baseline leg, always as the checker or the CPU baseline,
// never as part of the HIP product path.
//
// It follows the reference's CPU modules function by function:
//   * numerics            src/cpu/kernels/mod.rs:777-796, 2218-2245,
//                         2288-2313, 2365-2403
//   * conv / pool / deconv src/cpu/ops.rs:385-826, 1188-1326, 1480-1607
//   * layers              src/cpu/backend.rs:443-816, 1088-1370
//   * models              src/cpu/model.rs (cited per function below)
//   * preprocessing       src/preprocess.rs:78-123,
//                         src/preprocess/kernels.rs:10-18, 94-170
// Layout is NCHW float32 like the reference.  Built with -ffp-contract=off so
// that `a * b + c` rounds twice, as Rust does; every `mul_add` of the
// reference is an explicit std::fma here.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>
#include <omp.h>

namespace {

thread_local std::string g_error;

[[noreturn]] void fail(const std::string& msg) { throw std::runtime_error(msg); }
#define ENSURE(cond, msg) \
  do {                    \
    if (!(cond)) fail(msg); \
  } while (0)

// ---------------------------------------------------------------- tensors

struct Tensor {
  std::vector<int> shape;
  std::vector<float> v;
  Tensor() = default;
  Tensor(std::vector<int> s) : shape(std::move(s)) { v.assign(count(), 0.0f); }
  Tensor(std::vector<int> s, std::vector<float> d) : shape(std::move(s)), v(std::move(d)) {}
  size_t count() const {
    size_t n = 1;
    for (int d : shape) n *= (size_t)d;
    return n;
  }
  int n() const { return shape[0]; }
  int c() const { return shape[1]; }
  int h() const { return shape[2]; }
  int w() const { return shape[3]; }
  float* data() { return v.data(); }
  const float* data() const { return v.data(); }
};

// ---------------------------------------------------------------- test hooks
// Two switches that only tests turn on, both off by default:
//  * tracing records named intermediate tensors (block, neck, head and
//    encoder outputs), so a test can check one module's output in closed
//    form for weights it constructed;
//  * a fault plants one wiring mistake in the model composition, so a test
//    can show that its checks catch that mistake.
bool g_tracing = false;
std::map<std::string, Tensor> g_trace;
int g_fault = 0;

enum Fault {
  FAULT_NONE = 0,
  FAULT_LCNET_RESIDUAL_FROM_BLOCK_INPUT,  // residual adds the block input, not the post-token/SE tensor
  FAULT_LCNET_SE_GATE_FIFTH,              // LCNet SE gate hard-sigmoid(x/5 + 0.5)
  FAULT_NECK_SE_GATE_SIXTH,               // neck SE gate hard-sigmoid(x/6 + 0.5)
  FAULT_NECK_CONCAT_SHALLOW_FIRST,        // FPN / medium-neck concat [f0, f1 up2, f2 up4, f3 up8]
  FAULT_MISSING_GELU,                     // channel_conv1 without GELU
  FAULT_HEAD_BN_INPUT_AXIS,               // conv_up BN folded over the input-channel axis
  FAULT_SVTR_SKIP_BEFORE_NORM,            // LightSVTR: LN(seq + skip) instead of LN(seq) + skip
  FAULT_RECBLOCK_RESIDUAL_NORMED,         // RecBlock residual adds LN1(x) instead of x
  FAULT_QKV_HEAD_MAJOR,                   // qkv viewed as [heads, 3, hd] instead of [3, heads, hd]
  FAULT_TINY_HEAD_NO_HSWISH1,             // tiny recognizer head: no hardswish after conv1
  FAULT_NECK_SE_PLAIN_GATE,               // FPN residual SE as x * g instead of x + x * g
  FAULT_STEM_CONCAT_SWAPPED,              // large stem concat [branch, pooled]
  FAULT_INTRACLASS_ROW_COLUMN_SWAPPED,    // k x 1 kernel added into the centre row, 1 x k into the column
  FAULT_PAN_FROM_PROJECTION,              // bottom-up adds pan(projection[i-1]) instead of pan(bottom_up[i-1])
  FAULT_TOPDOWN_NOT_CASCADED,             // top-down adds the level above before its own update
  FAULT_ATTENTION_SCALE_HIDDEN,           // scores scaled by hidden^-0.5 instead of head_dim^-0.5
  FAULT_SMALL_STEM_NO_GELU,               // tiny recognizer stem without GELU
  FAULT_COUNT
};

inline bool fault(int f) { return g_fault == f; }

// bf16 storage emulation (tests of the bf16 path): when on, the values a
// bf16 plan rounds to bf16 (nearest even) are rounded where they are
// produced, and so are the weights it feeds to the matrix cores (dense convs
// and linear layers, depthwise 5x5 and wider, the head's transposed conv;
// after BN folding); sums, SE gates, LayerNorm parameters, biases and the
// outputs stay fp32.  A sum that a bf16 plan forms in one kernel epilogue
// (a residual or upsampled add after a conv or linear layer, the LightSVTR
// skip after the final LayerNorm, the FPN's x + x*g + up2(upper)) is rounded
// once, after the add.  Every rounding point is named (the value, or "W"
// and the layer for weights) and logged, so a test can compare the list
// with the plan's own.  The error of this emulation against the fp32
// oracle is the yardstick of the bf16 path's tolerances.
bool g_bf16 = false;
std::vector<std::string> g_bf16_log;

// Summation order (tests only): with g_reverse_sums the matrix products,
// depthwise convs and attention sums accumulate their terms last to first.
// Under the bf16 emulation, the spread between the two orders measures how
// far fp32 summation order alone moves outputs of a bf16-storage network.
bool g_reverse_sums = false;

inline float round_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return f;
  u = ((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16) << 16;
  memcpy(&f, &u, 4);
  return f;
}

// Rounds t (the value `name`) in place when the emulation is on; returns it.
Tensor& bf(Tensor& t, const std::string& name) {
  if (g_bf16) {
    g_bf16_log.push_back("A " + name);
    for (float& v : t.v) v = round_bf16(v);
  }
  return t;
}

// w (the weights of layer `name`) itself, or with the emulation on a
// bf16-rounded copy of it held in tmp.
const Tensor& bf_weights(const Tensor& w, Tensor& tmp, const std::string& name) {
  if (!g_bf16) return w;
  g_bf16_log.push_back("W " + name);
  tmp = w;
  for (float& v : tmp.v) v = round_bf16(v);
  return tmp;
}

void trace(const std::string& name, const Tensor& t) {
  if (g_tracing) g_trace[name] = t;
}

// ---------------------------------------------------------------- safetensors
// Minimal reader: 8-byte little-endian header length, JSON header, raw data.
// F32 only, as the reference CPU loader (src/cpu/weights.rs:14-47).

struct JsonReader {
  const std::string& s;
  size_t i = 0;
  explicit JsonReader(const std::string& text) : s(text) {}
  void ws() {
    while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t')) ++i;
  }
  char peek() {
    ws();
    ENSURE(i < s.size(), "safetensors header truncated");
    return s[i];
  }
  void expect(char c) {
    ENSURE(peek() == c, std::string("safetensors header: expected ") + c);
    ++i;
  }
  std::string str() {
    expect('"');
    std::string out;
    while (i < s.size() && s[i] != '"') {
      if (s[i] == '\\') {
        ++i;
        ENSURE(i < s.size(), "bad escape");
        out.push_back(s[i]);
      } else {
        out.push_back(s[i]);
      }
      ++i;
    }
    ENSURE(i < s.size(), "unterminated string");
    ++i;
    return out;
  }
  double num() {
    ws();
    size_t j = i;
    while (j < s.size() && (isdigit((unsigned char)s[j]) || s[j] == '-' || s[j] == '+' || s[j] == '.' ||
                            s[j] == 'e' || s[j] == 'E'))
      ++j;
    ENSURE(j > i, "expected number");
    double d = std::stod(s.substr(i, j - i));
    i = j;
    return d;
  }
  void skip() {
    char c = peek();
    if (c == '"') {
      str();
    } else if (c == '{') {
      ++i;
      if (peek() == '}') { ++i; return; }
      for (;;) {
        str();
        expect(':');
        skip();
        if (peek() == ',') { ++i; continue; }
        expect('}');
        return;
      }
    } else if (c == '[') {
      ++i;
      if (peek() == ']') { ++i; return; }
      for (;;) {
        skip();
        if (peek() == ',') { ++i; continue; }
        expect(']');
        return;
      }
    } else if (s.compare(i, 4, "true") == 0 || s.compare(i, 4, "null") == 0) {
      i += 4;
    } else if (s.compare(i, 5, "false") == 0) {
      i += 5;
    } else {
      num();
    }
  }
};

struct Weights {
  std::map<std::string, Tensor> t;

  static Weights load(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    ENSURE(f.good(), "read weights " + path);
    std::vector<char> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    ENSURE(bytes.size() >= 8, "safetensors file too short");
    uint64_t hlen = 0;
    memcpy(&hlen, bytes.data(), 8);
    ENSURE(8 + hlen <= bytes.size(), "safetensors header exceeds file");
    std::string header(bytes.data() + 8, bytes.data() + 8 + hlen);
    size_t base = 8 + hlen;
    Weights w;
    JsonReader r(header);
    r.expect('{');
    if (r.peek() == '}') return w;
    for (;;) {
      std::string name = r.str();
      r.expect(':');
      if (name == "__metadata__") {
        r.skip();
      } else {
        std::string dtype;
        std::vector<int> shape;
        size_t start = 0, end = 0;
        r.expect('{');
        for (;;) {
          std::string key = r.str();
          r.expect(':');
          if (key == "dtype") {
            dtype = r.str();
          } else if (key == "shape") {
            r.expect('[');
            if (r.peek() == ']') {
              ++r.i;
            } else {
              for (;;) {
                shape.push_back((int)r.num());
                if (r.peek() == ',') { ++r.i; continue; }
                r.expect(']');
                break;
              }
            }
          } else if (key == "data_offsets") {
            r.expect('[');
            start = (size_t)r.num();
            r.expect(',');
            end = (size_t)r.num();
            r.expect(']');
          } else {
            r.skip();
          }
          if (r.peek() == ',') { ++r.i; continue; }
          r.expect('}');
          break;
        }
        ENSURE(dtype == "F32", "tensor " + name + " has dtype " + dtype + "; expected F32");
        Tensor t(shape);
        ENSURE(end >= start && base + end <= bytes.size(), "tensor " + name + " range exceeds file");
        ENSURE(end - start == t.count() * 4, "tensor " + name + " byte length mismatch");
        memcpy(t.data(), bytes.data() + base + start, end - start);
        w.t.emplace(name, std::move(t));
      }
      if (r.peek() == ',') { ++r.i; continue; }
      r.expect('}');
      break;
    }
    return w;
  }

  // VarBuilder::get with shape validation (src/cpu/weights.rs:77-95).
  Tensor get(const std::string& name, std::vector<int> shape) const {
    auto it = t.find(name);
    ENSURE(it != t.end(), "tensor \"" + name + "\" was not found");
    ENSURE(it->second.shape == shape, "tensor \"" + name + "\" has an unexpected shape");
    return it->second;
  }
};

// ---------------------------------------------------------------- numerics

enum Act { ACT_NONE = 0, ACT_RELU, ACT_GELU, ACT_SILU, ACT_HSIG6, ACT_HSIG5, ACT_HSWISH, ACT_SIGMOID };

// Abramowitz-Stegun 7.1.26 (src/cpu/kernels/mod.rs:2392-2403).
float erf_as(float value) {
  float sign = value < 0.0f ? -1.0f : 1.0f;
  float x = std::fabs(value);
  float t = 1.0f / std::fma(x, 0.3275911f, 1.0f);
  float poly = t * (0.2548296f + t * (-0.28449672f + t * (1.4214138f + t * (-1.4531521f + t * 1.0614054f))));
  return sign * (1.0f - poly * std::exp(-x * x));
}

// UnaryOperation::apply (src/cpu/kernels/mod.rs:2376-2390).
float apply_act(int act, float v) {
  switch (act) {
    case ACT_RELU: return std::fmax(v, 0.0f);
    case ACT_GELU: return 0.5f * v * (1.0f + erf_as(v * 0.70710678118654752f));
    case ACT_SILU: return v / (1.0f + std::exp(-v));
    case ACT_HSIG6: return std::clamp(std::fma(v, 1.0f / 6.0f, 0.5f), 0.0f, 1.0f);
    case ACT_HSIG5: return std::clamp(std::fma(v, 0.2f, 0.5f), 0.0f, 1.0f);
    case ACT_HSWISH: return v * std::clamp(v / 6.0f + 0.5f, 0.0f, 1.0f);
    case ACT_SIGMOID: return 1.0f / (1.0f + std::exp(-v));
    default: return v;
  }
}

void act_in_place(Tensor& t, int act) {
  if (act == ACT_NONE) return;
  float* p = t.data();
  long n = (long)t.count();
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) p[i] = apply_act(act, p[i]);
}

// softmax_in_place (src/cpu/kernels/mod.rs:2218-2245).
void softmax_row(float* v, int n) {
  float m = -INFINITY;
  for (int i = 0; i < n; ++i) m = std::fmax(m, v[i]);
  float sum = 0.0f;
  for (int i = 0; i < n; ++i) {
    v[i] = std::exp(v[i] - m);
    sum += v[i];
  }
  float r = 1.0f / sum;
  for (int i = 0; i < n; ++i) v[i] *= r;
}

// layer_norm_in_place (src/cpu/kernels/mod.rs:2288-2313).
void layer_norm_row(float* v, const float* w, const float* b, int n, float eps) {
  float sum = 0.0f;
  for (int i = 0; i < n; ++i) sum += v[i];
  float mean = sum / (float)n;
  float var = 0.0f;
  for (int i = 0; i < n; ++i) {
    float c = v[i] - mean;
    var += c * c;
  }
  var /= (float)n;
  float inv = 1.0f / std::sqrt(var + eps);
  for (int i = 0; i < n; ++i) v[i] = std::fma(v[i] - mean, inv * w[i], b[i]);
}

// residual_mul_in_place: two roundings fma(fma(v,g,0),1,v)
// (src/cpu/kernels/mod.rs:777-796).
inline float residual_mul(float v, float g) {
  float scaled = std::fma(v, g, 0.0f);
  return std::fma(scaled, 1.0f, v);
}

// ---------------------------------------------------------------- GEMM
// C[M][N] = A[M][K] * B[K][N] (+bias[m]) then activation.  B has row stride
// ldb.  Accumulation is FMA, as the reference kernels.
void gemm(float* C, const float* A, const float* B, int M, int K, int N, long ldb, const float* bias,
          int act) {
  const int NB = 256, MB = 8;
  int mblocks = (M + MB - 1) / MB, nblocks = (N + NB - 1) / NB;
#pragma omp parallel for schedule(dynamic) collapse(2)
  for (int mb = 0; mb < mblocks; ++mb) {
    for (int nb = 0; nb < nblocks; ++nb) {
      int m0 = mb * MB, m1 = std::min(M, m0 + MB);
      int n0 = nb * NB, n1 = std::min(N, n0 + NB);
      int nn = n1 - n0;
      float acc[MB][NB];
      for (int m = m0; m < m1; ++m)
        for (int j = 0; j < nn; ++j) acc[m - m0][j] = 0.0f;
      for (int kk = 0; kk < K; ++kk) {
        const int k = g_reverse_sums ? K - 1 - kk : kk;
        const float* b = B + (long)k * ldb + n0;
        for (int m = m0; m < m1; ++m) {
          float a = A[(long)m * K + k];
          float* ac = acc[m - m0];
          for (int j = 0; j < nn; ++j) ac[j] = std::fma(a, b[j], ac[j]);
        }
      }
      for (int m = m0; m < m1; ++m) {
        float bb = bias ? bias[m] : 0.0f;
        float* c = C + (long)m * N + n0;
        for (int j = 0; j < nn; ++j) c[j] = apply_act(act, acc[m - m0][j] + bb);
      }
    }
  }
}

// ---------------------------------------------------------------- ops

// ops::conv (src/cpu/ops.rs:385-826): NCHW, pads [top, left, bottom, right],
// output = floor((in + pt + pb - k) / s) + 1, groups 1 or depthwise.
Tensor conv2d(const Tensor& x, const Tensor& W, const float* bias, int sh, int sw, const int pads[4], int groups,
              int act) {
  int N = x.n(), C = x.c(), H = x.h(), Wd = x.w();
  int Co = W.shape[0], Cg = W.shape[1], kh = W.shape[2], kw = W.shape[3];
  ENSURE(C == Cg * groups, "Conv input channels do not match weights and groups");
  int Ho = (H + pads[0] + pads[2] - kh) / sh + 1;
  int Wo = (Wd + pads[1] + pads[3] - kw) / sw + 1;
  Tensor y({N, Co, Ho, Wo});
  long P = (long)Ho * Wo;
  if (groups == 1) {
    int K = C * kh * kw;
    bool direct = kh == 1 && kw == 1 && sh == 1 && sw == 1 && pads[0] == 0 && pads[1] == 0 && pads[2] == 0 &&
                  pads[3] == 0;
    std::vector<float> col;
    if (!direct) col.resize((size_t)K * P);
    for (int n = 0; n < N; ++n) {
      const float* xin = x.data() + (size_t)n * C * H * Wd;
      const float* B = xin;
      if (!direct) {
#pragma omp parallel for schedule(static)
        for (int k = 0; k < K; ++k) {
          int c = k / (kh * kw), r = k % (kh * kw), ky = r / kw, kx = r % kw;
          float* dst = col.data() + (size_t)k * P;
          const float* src = xin + (size_t)c * H * Wd;
          for (int oy = 0; oy < Ho; ++oy) {
            int iy = oy * sh + ky - pads[0];
            for (int ox = 0; ox < Wo; ++ox) {
              int ix = ox * sw + kx - pads[1];
              dst[(long)oy * Wo + ox] = (iy >= 0 && iy < H && ix >= 0 && ix < Wd) ? src[(long)iy * Wd + ix] : 0.0f;
            }
          }
        }
        B = col.data();
      }
      gemm(y.data() + (size_t)n * Co * P, W.data(), B, Co, K, (int)P, P, bias, act);
    }
    return y;
  }
  ENSURE(groups == C && Co == C && Cg == 1, "only depthwise grouped convs are supported");
#pragma omp parallel for collapse(2) schedule(static)
  for (int n = 0; n < N; ++n) {
    for (int c = 0; c < C; ++c) {
      const float* src = x.data() + ((size_t)n * C + c) * H * Wd;
      const float* wk = W.data() + (size_t)c * kh * kw;
      float* dst = y.data() + ((size_t)n * C + c) * P;
      float bb = bias ? bias[c] : 0.0f;
      for (int oy = 0; oy < Ho; ++oy) {
        for (int ox = 0; ox < Wo; ++ox) {
          float acc = 0.0f;
          for (int kyy = 0; kyy < kh; ++kyy) {
            const int ky = g_reverse_sums ? kh - 1 - kyy : kyy;
            int iy = oy * sh + ky - pads[0];
            if (iy < 0 || iy >= H) continue;
            for (int kxx = 0; kxx < kw; ++kxx) {
              const int kx = g_reverse_sums ? kw - 1 - kxx : kxx;
              int ix = ox * sw + kx - pads[1];
              if (ix < 0 || ix >= Wd) continue;
              acc = std::fma(src[(long)iy * Wd + ix], wk[ky * kw + kx], acc);
            }
          }
          dst[(long)oy * Wo + ox] = apply_act(act, acc + bb);
        }
      }
    }
  }
  return y;
}

// ConvTranspose2d 2x2 stride 2, IOHW weight [Cin, Cout, 2, 2]
// (src/cpu/ops.rs:1232-1267, src/cpu/backend.rs:1088-1181).
Tensor conv_transpose2x2(const Tensor& x, const Tensor& W, const float* bias) {
  int N = x.n(), C = x.c(), H = x.h(), Wd = x.w();
  ENSURE(W.shape[0] == C && W.shape[2] == 2 && W.shape[3] == 2, "ConvTranspose weight shape");
  int Co = W.shape[1];
  Tensor y({N, Co, 2 * H, 2 * Wd});
  long P = (long)H * Wd;
  // Packed rows (o*4 + kidx) x Cin, as forward_2x2 does.
  std::vector<float> packed((size_t)Co * 4 * C);
  for (int o = 0; o < Co; ++o)
    for (int k = 0; k < 4; ++k)
      for (int c = 0; c < C; ++c) packed[((size_t)o * 4 + k) * C + c] = W.v[((size_t)c * Co + o) * 4 + k];
  std::vector<float> tile((size_t)Co * 4 * P);
  for (int n = 0; n < N; ++n) {
    gemm(tile.data(), packed.data(), x.data() + (size_t)n * C * P, Co * 4, C, (int)P, P, nullptr, ACT_NONE);
#pragma omp parallel for schedule(static)
    for (int o = 0; o < Co; ++o) {
      float b = bias ? bias[o] : 0.0f;
      float* out = y.data() + ((size_t)n * Co + o) * 4 * P;
      const float* t = tile.data() + (size_t)o * 4 * P;
      for (int iy = 0; iy < H; ++iy)
        for (int ix = 0; ix < Wd; ++ix) {
          long i = (long)iy * Wd + ix;
          long top = (long)(2 * iy) * (2 * Wd) + 2 * ix;
          long bot = top + 2 * Wd;
          out[top] = t[i] + b;
          out[top + 1] = t[P + i] + b;
          out[bot] = t[2 * P + i] + b;
          out[bot + 1] = t[3 * P + i] + b;
        }
    }
  }
  return y;
}

// Max pool 2x2, stride 1, pads (0,0,1,1): windows past the bottom/right edge
// are clipped; NaN is ignored by f32::max (src/cpu/ops.rs:1520-1535).
Tensor max_pool_2x2_same(const Tensor& x) {
  Tensor y(x.shape);
  int H = x.h(), W = x.w();
  long planes = (long)x.n() * x.c();
#pragma omp parallel for schedule(static)
  for (long p = 0; p < planes; ++p) {
    const float* s = x.data() + p * H * W;
    float* d = y.data() + p * H * W;
    for (int yy = 0; yy < H; ++yy)
      for (int xx = 0; xx < W; ++xx) {
        float m = -INFINITY;
        for (int dy = 0; dy < 2; ++dy)
          for (int dx = 0; dx < 2; ++dx) {
            int iy = yy + dy, ix = xx + dx;
            if (iy < H && ix < W) m = std::fmax(m, s[(long)iy * W + ix]);
          }
        d[(long)yy * W + xx] = m;
      }
  }
  return y;
}

// Average pool, kernel [3,2], stride [3,2], no pad, count_include_pad=false
// (src/cpu/ops.rs:1537-1604).
Tensor avg_pool_3x2(const Tensor& x, const std::string& name = "pool") {
  int H = x.h(), W = x.w();
  int Ho = (H - 3) / 3 + 1, Wo = (W - 2) / 2 + 1;
  Tensor y({x.n(), x.c(), Ho, Wo});
  long planes = (long)x.n() * x.c();
#pragma omp parallel for schedule(static)
  for (long p = 0; p < planes; ++p) {
    const float* s = x.data() + p * H * W;
    float* d = y.data() + p * Ho * Wo;
    for (int oy = 0; oy < Ho; ++oy)
      for (int ox = 0; ox < Wo; ++ox) {
        float v = 0.0f;
        for (int ky = 0; ky < 3; ++ky)
          for (int kx = 0; kx < 2; ++kx) v = v + s[(long)(oy * 3 + ky) * W + ox * 2 + kx];
        d[(long)oy * Wo + ox] = v / 6.0f;
      }
  }
  return bf(y, name);
}

// global_average_pool: mean over the plane (src/cpu/ops.rs:1480-1495).
Tensor global_mean(const Tensor& x) {
  Tensor y({x.n(), x.c(), 1, 1});
  long plane = (long)x.h() * x.w();
  long planes = (long)x.n() * x.c();
#pragma omp parallel for schedule(static)
  for (long p = 0; p < planes; ++p) {
    const float* s = x.data() + p * plane;
    float sum = 0.0f;
    for (long i = 0; i < plane; ++i) sum += s[i];
    y.v[p] = sum / (float)plane;
  }
  return y;
}

Tensor add(const Tensor& a, const Tensor& b, const std::string& name = "") {
  ENSURE(a.shape == b.shape, "add shape mismatch");
  Tensor y(a.shape);
  long n = (long)a.count();
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) y.v[i] = a.v[i] + b.v[i];
  return bf(y, name);
}

// x * gate[n, c] (plain SE, src/cpu/model.rs:487-492).
Tensor mul_gate(const Tensor& x, const Tensor& g, const std::string& name = "") {
  Tensor y(x.shape);
  long plane = (long)x.h() * x.w();
  long planes = (long)x.n() * x.c();
#pragma omp parallel for schedule(static)
  for (long p = 0; p < planes; ++p)
    for (long i = 0; i < plane; ++i) y.v[p * plane + i] = x.v[p * plane + i] * g.v[p];
  return bf(y, name);
}

// into_residual_mul (src/cpu/backend.rs:180-199).
// With `round` false the result stays fp32 (an add follows in the same
// kernel of a bf16 plan).
Tensor residual_mul_gate(const Tensor& x, const Tensor& g, const std::string& name = "", bool round = true) {
  Tensor y(x.shape);
  long plane = (long)x.h() * x.w();
  long planes = (long)x.n() * x.c();
#pragma omp parallel for schedule(static)
  for (long p = 0; p < planes; ++p)
    for (long i = 0; i < plane; ++i) y.v[p * plane + i] = residual_mul(x.v[p * plane + i], g.v[p]);
  return round ? bf(y, name) : y;
}

// upsample_add_nchw: feature[y][x] += upper[y/s][x/s] (src/cpu/model.rs:1265-1320).
Tensor upsample_add(Tensor feature, const Tensor& upper, int s, const std::string& name = "") {
  ENSURE(feature.n() == upper.n() && feature.c() == upper.c() && feature.h() == upper.h() * s &&
             feature.w() == upper.w() * s,
         "upsample-add shape mismatch");
  int H = feature.h(), W = feature.w(), uh = upper.h(), uw = upper.w();
  long planes = (long)feature.n() * feature.c();
#pragma omp parallel for schedule(static)
  for (long p = 0; p < planes; ++p)
    for (int y = 0; y < H; ++y)
      for (int x = 0; x < W; ++x)
        feature.v[(p * H + y) * W + x] += upper.v[(p * uh + y / s) * uw + x / s];
  return bf(feature, name);
}

// upsample_and_cat_nchw: nearest integer upsample then channel concat
// (src/cpu/model.rs:1322-1417).
Tensor upsample_cat(const std::vector<Tensor>& fs, const std::vector<int>& scales) {
  ENSURE(!fs.empty() && fs.size() == scales.size(), "upsample-cat arguments");
  int N = fs[0].n(), H = fs[0].h() * scales[0], W = fs[0].w() * scales[0];
  int C = 0;
  for (size_t i = 0; i < fs.size(); ++i) {
    ENSURE(fs[i].n() == N && fs[i].h() * scales[i] == H && fs[i].w() * scales[i] == W, "upsample-cat mismatch");
    C += fs[i].c();
  }
  Tensor y({N, C, H, W});
  for (int n = 0; n < N; ++n) {
    int oc = 0;
    for (size_t i = 0; i < fs.size(); ++i) {
      const Tensor& f = fs[i];
      int s = scales[i];
#pragma omp parallel for schedule(static)
      for (int c = 0; c < f.c(); ++c)
        for (int yy = 0; yy < H; ++yy)
          for (int xx = 0; xx < W; ++xx)
            y.v[(((size_t)n * C + oc + c) * H + yy) * W + xx] =
                f.v[(((size_t)n * f.c() + c) * f.h() + yy / s) * f.w() + xx / s];
      oc += f.c();
    }
  }
  return y;
}

// Linear::run: y = x W^T + b, optional activation / row softmax
// (src/cpu/backend.rs:1292-1370).
// `name` names the layer (its weights) and its output value; with `round`
// false the output stays fp32 (an add follows in the same kernel of a bf16
// plan).
Tensor linear(const Tensor& x, const Tensor& W_, const Tensor* b, int act, bool softmax, const std::string& name = "",
              bool round = true) {
  Tensor tmp;
  const Tensor& W = bf_weights(W_, tmp, name);
  int K = W.shape[1], M = W.shape[0];
  ENSURE(x.shape.back() == K, "Linear input feature count");
  long rows = (long)x.count() / K;
  std::vector<int> shape = x.shape;
  shape.back() = M;
  Tensor y(shape);
#pragma omp parallel for schedule(dynamic, 4)
  for (long r = 0; r < rows; ++r) {
    const float* xi = x.data() + r * K;
    float* yo = y.data() + r * M;
    for (int m = 0; m < M; ++m) {
      const float* wr = W.data() + (size_t)m * K;
      float acc = 0.0f;
      for (int kk = 0; kk < K; ++kk) {
        const int k = g_reverse_sums ? K - 1 - kk : kk;
        acc = std::fma(xi[k], wr[k], acc);
      }
      yo[m] = apply_act(act, acc + (b ? b->v[m] : 0.0f));
    }
    if (softmax) softmax_row(yo, M);
  }
  return softmax || !round ? y : bf(y, name);
}

Tensor layer_norm(const Tensor& x, const Tensor& w, const Tensor& b, float eps, const std::string& name = "",
                  bool round = true) {
  int F = w.shape[0];
  Tensor y = x;
  long rows = (long)x.count() / F;
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; ++r) layer_norm_row(y.data() + r * F, w.data(), b.data(), F, eps);
  return round ? bf(y, name) : y;
}

// ---------------------------------------------------------------- layers

// fold_batch_norm (src/cpu/model.rs:371-407): s = g / sqrt(var + 1e-5),
// W' = W s per output channel, b' = (b - mean) s + beta.
void fold_bn(Tensor& W, std::vector<float>& bias, const Weights& wt, const std::string& norm, int channels) {
  Tensor g = wt.get(norm + ".weight", {channels});
  Tensor be = wt.get(norm + ".bias", {channels});
  Tensor mu = wt.get(norm + ".running_mean", {channels});
  Tensor var = wt.get(norm + ".running_var", {channels});
  if (bias.empty()) bias.assign(channels, 0.0f);
  size_t row = W.count() / channels;
  for (int c = 0; c < channels; ++c) {
    float s = g.v[c] / std::sqrt(var.v[c] + 1e-5f);
    for (size_t i = 0; i < row; ++i) W.v[c * row + i] *= s;
    bias[c] = (bias[c] - mu.v[c]) * s + be.v[c];
  }
}

struct Conv {
  Tensor W;
  std::vector<float> b;
  int sh = 1, sw = 1, pads[4] = {0, 0, 0, 0}, groups = 1;
  int act = ACT_NONE;
  bool fp32_only = false;  // SE 1x1 convs: fp32 weights and outputs in every plan
  std::string name;        // module path: names the weights and the output value
  // With `round` false the output stays fp32: an add follows in the same
  // kernel of a bf16 plan.
  Tensor forward(const Tensor& x, int a = -1, bool round = true) const {
    // Matrix-core layers (dense convs, depthwise 5x5 and wider) take bf16
    // weights in a bf16 plan.
    const bool mfma = groups == 1 || (W.shape[2] >= 5 && W.shape[3] >= 5);
    Tensor tmp;
    const Tensor& w = !fp32_only && mfma ? bf_weights(W, tmp, name) : W;
    Tensor y = conv2d(x, w, b.empty() ? nullptr : b.data(), sh, sw, pads, groups, a < 0 ? act : a);
    return fp32_only || !round ? y : bf(y, name);
  }
};

// Conv2d::load (src/cpu/model.rs:89-107).
Conv load_conv(const Weights& wt, const std::string& p, int ci, int co, int kh, int kw, int sh, int sw,
               std::vector<int> pads, bool bias, int groups, int act = ACT_NONE) {
  Conv c;
  c.name = p;
  c.W = wt.get(p + ".weight", {co, ci / groups, kh, kw});
  if (bias) c.b = wt.get(p + ".bias", {co}).v;
  c.sh = sh;
  c.sw = sw;
  for (int i = 0; i < 4; ++i) c.pads[i] = pads[i];
  c.groups = groups;
  c.act = act;
  return c;
}

// ConvBnAct::load / Conv2d::load_bn (src/cpu/model.rs:110-131, 409-454).
Conv load_conv_bn(const Weights& wt, const std::string& p, int ci, int co, int kh, int kw, int sh, int sw,
                  std::vector<int> pads, bool bias, int groups, const std::string& norm, int act) {
  Conv c = load_conv(wt, p + ".convolution", ci, co, kh, kw, sh, sw, pads, bias, groups, act);
  c.name = p;
  fold_bn(c.W, c.b, wt, p + "." + norm, co);
  return c;
}

// SqueezeExcitation (src/cpu/model.rs:456-493) and
// VariantSqueezeExcitation::attention (:1069-1105).
struct SE {
  Conv reduce, expand;
  int gate_act = ACT_HSIG6;
  Tensor gate(const Tensor& x) const {
    const_cast<Conv&>(reduce).fp32_only = true;
    const_cast<Conv&>(expand).fp32_only = true;
    Tensor pooled = global_mean(x);
    Tensor r = reduce.forward(pooled, ACT_RELU);
    Tensor e = expand.forward(r, ACT_NONE);
    act_in_place(e, gate_act);
    return e;
  }
};

// LcNetBlock (src/cpu/model.rs:509-603): token conv (plain bias when
// residual, BN-folded otherwise) -> [SE x*g] -> 1x1 C->2C GELU -> 1x1 2C->C'
// -> + (post-token/SE tensor) when residual.
struct LcNetBlock {
  Conv token, conv1, conv2;
  bool has_se = false, residual = false;
  SE se;
  Tensor forward(const Tensor& x) const {
    Tensor t = token.forward(x);
    if (has_se) t = mul_gate(t, se.gate(t), conv1.name + ".gated");
    Tensor h = conv1.forward(t, fault(FAULT_MISSING_GELU) ? ACT_NONE : ACT_GELU);
    if (!residual) return conv2.forward(h, ACT_NONE);
    Tensor o = conv2.forward(h, ACT_NONE, false);
    return add(fault(FAULT_LCNET_RESIDUAL_FROM_BLOCK_INPUT) ? x : t, o, conv2.name);
  }
};

struct BlockSpec {
  int ci, co, sh, sw;
  bool se;
};

LcNetBlock load_block(const Weights& wt, const std::string& p, BlockSpec s) {
  LcNetBlock b;
  b.residual = s.ci == s.co && s.sh == 1 && s.sw == 1;
  if (b.residual) {
    b.token = load_conv(wt, p + ".token_conv", s.ci, s.co, 3, 3, s.sh, s.sw, {1, 1, 1, 1}, true, s.ci);
  } else {
    b.token = load_conv_bn(wt, p + ".token_conv", s.ci, s.ci, 3, 3, s.sh, s.sw, {1, 1, 1, 1}, false, s.ci,
                           "normalization", ACT_NONE);
  }
  b.has_se = s.se;
  if (s.se) {
    std::string q = p + ".token_squeeze_excitation.convolutions";
    b.se.reduce = load_conv(wt, q + ".0", s.ci, s.ci / 4, 1, 1, 1, 1, {0, 0, 0, 0}, true, 1);
    b.se.expand = load_conv(wt, q + ".2", s.ci / 4, s.ci, 1, 1, 1, 1, {0, 0, 0, 0}, true, 1);
    b.se.gate_act = fault(FAULT_LCNET_SE_GATE_FIFTH) ? ACT_HSIG5 : ACT_HSIG6;
  }
  b.conv1 = load_conv_bn(wt, p + ".channel_conv1", s.ci, s.ci * 2, 1, 1, 1, 1, {0, 0, 0, 0}, false, 1,
                         "normalization", ACT_NONE);
  b.conv2 = load_conv_bn(wt, p + ".channel_conv2", s.ci * 2, s.co, 1, 1, 1, 1, {0, 0, 0, 0}, false, 1,
                         "normalization", ACT_NONE);
  return b;
}

// LcNetBackbone with LargeStem (src/cpu/model.rs:626-693) or SmallStem
// (:695-733).
struct Backbone {
  bool large = true;
  Conv stem1, stem2a, stem2b, stem3, stem4;  // large
  Conv conv1, conv2;                         // small
  std::vector<std::vector<LcNetBlock>> stages;

  Tensor stem(const Tensor& x) const {
    if (!large)
      return conv2.forward(conv1.forward(x, fault(FAULT_SMALL_STEM_NO_GELU) ? ACT_NONE : ACT_GELU), ACT_NONE);
    Tensor e = stem1.forward(x);
    Tensor br = stem2b.forward(stem2a.forward(e));
    Tensor pooled = max_pool_2x2_same(e);
    Tensor merged = fault(FAULT_STEM_CONCAT_SWAPPED) ? upsample_cat({br, pooled}, {1, 1})
                                                     : upsample_cat({pooled, br}, {1, 1});
    return stem4.forward(stem3.forward(merged));
  }
  std::vector<Tensor> forward(const Tensor& x) const {
    Tensor h = stem(x);
    trace("stem", h);
    std::vector<Tensor> outs;
    for (size_t s = 0; s < stages.size(); ++s) {
      for (size_t b = 0; b < stages[s].size(); ++b) {
        h = stages[s][b].forward(h);
        trace("block" + std::to_string(s) + "." + std::to_string(b), h);
      }
      outs.push_back(h);
    }
    return outs;
  }
};

Backbone load_backbone(const Weights& wt, int mid, int out, const std::vector<std::vector<BlockSpec>>& specs,
                       bool large) {
  Backbone bb;
  bb.large = large;
  std::string p = "model.backbone.encoder.convolution";
  if (large) {
    bb.stem1 = load_conv_bn(wt, p + ".stem1", 3, mid, 3, 3, 2, 2, {1, 1, 1, 1}, false, 1, "normalization", ACT_RELU);
    bb.stem2a = load_conv_bn(wt, p + ".stem2a", mid, mid / 2, 2, 2, 1, 1, {0, 0, 1, 1}, false, 1, "normalization",
                             ACT_RELU);
    bb.stem2b = load_conv_bn(wt, p + ".stem2b", mid / 2, mid, 2, 2, 1, 1, {0, 0, 1, 1}, false, 1, "normalization",
                             ACT_RELU);
    bb.stem3 = load_conv_bn(wt, p + ".stem3", mid * 2, mid, 3, 3, 2, 2, {1, 1, 1, 1}, false, 1, "normalization",
                            ACT_RELU);
    bb.stem4 = load_conv_bn(wt, p + ".stem4", mid, out, 1, 1, 1, 1, {0, 0, 0, 0}, false, 1, "normalization",
                            ACT_RELU);
  } else {
    bb.conv1 = load_conv_bn(wt, p + ".conv1", 3, mid, 3, 3, 2, 2, {1, 1, 1, 1}, false, 1, "normalization", ACT_NONE);
    bb.conv2 = load_conv_bn(wt, p + ".conv2", mid, out, 3, 3, 2, 2, {1, 1, 1, 1}, false, 1, "normalization", ACT_NONE);
  }
  for (size_t s = 0; s < specs.size(); ++s) {
    std::vector<LcNetBlock> blocks;
    for (size_t b = 0; b < specs[s].size(); ++b)
      blocks.push_back(load_block(wt, "model.backbone.encoder.blocks." + std::to_string(s) + ".blocks." +
                                          std::to_string(b),
                                  specs[s][b]));
    bb.stages.push_back(std::move(blocks));
  }
  return bb;
}

// detector_stages_for_channels (src/cpu/model.rs:1648-1673).
std::vector<std::vector<BlockSpec>> detector_stages(int s1, int s2, int s3, int s4) {
  return {
      {{s1, s1, 1, 1, true}, {s1, s1, 1, 1, false}},
      {{s1, s2, 2, 2, false}, {s2, s2, 1, 1, true}, {s2, s2, 1, 1, false}},
      {{s2, s3, 2, 2, false}, {s3, s3, 1, 1, true}, {s3, s3, 1, 1, false}, {s3, s3, 1, 1, true},
       {s3, s3, 1, 1, false}},
      {{s3, s4, 2, 2, false}, {s4, s4, 1, 1, true}, {s4, s4, 1, 1, false}},
  };
}

// recognizer stage tables (src/cpu/model.rs:2057-2122).
std::vector<std::vector<BlockSpec>> recognizer_stages(int size) {
  auto alt = [](int c) {
    std::vector<BlockSpec> v;
    for (int i = 0; i < 6; ++i) v.push_back({c, c, 1, 1, i % 2 == 0});
    return v;
  };
  if (size == 0) {  // medium
    std::vector<BlockSpec> s3 = {{256, 512, 2, 1, false}};
    for (auto b : alt(512)) s3.push_back(b);
    return {{{128, 128, 1, 1, true}},
            {{128, 256, 1, 1, false}, {256, 256, 1, 1, false}, {256, 256, 1, 1, true}},
            s3,
            {{512, 768, 2, 1, false}, {768, 768, 1, 1, true}, {768, 768, 1, 1, false}}};
  }
  if (size == 1) {  // small
    std::vector<BlockSpec> s3 = {{96, 192, 2, 1, false}};
    for (auto b : alt(192)) s3.push_back(b);
    return {{{96, 96, 1, 1, true}},
            {{96, 96, 1, 1, false}, {96, 96, 1, 1, false}},
            s3,
            {{192, 384, 2, 1, false}, {384, 384, 1, 1, true}, {384, 384, 1, 1, false}}};
  }
  return {{{48, 48, 1, 1, true}},
          {{48, 48, 1, 1, false}},
          {{48, 96, 2, 1, false}, {96, 96, 1, 1, true}, {96, 96, 1, 1, false}},
          {{96, 160, 2, 1, false}, {160, 160, 1, 1, true}, {160, 160, 1, 1, false}, {160, 160, 1, 1, false}}};
}

// factor_rank_one_conv_weight (src/cpu/model.rs:221-369): per input channel,
// four power iterations in f64 on the O x K^2 matrix, then the separability
// check (max error <= 1e-5 max|W| + 1e-12, relative Frobenius <= 1e-6).
void factor_rank_one(const Tensor& W, int ci, int co, int k, Tensor& dw, Tensor& pw) {
  ENSURE(k > 0 && k % 2 == 1, "rank-one convolution kernel must be positive and odd");
  const float* src = W.data();
  for (size_t i = 0; i < W.count(); ++i) ENSURE(std::isfinite(src[i]), "rank-one weight has non-finite values");
  int sp = k * k;
  dw = Tensor({ci, 1, k, k});
  pw = Tensor({co, ci, 1, 1});
  std::vector<double> dir(sp), scales(co);
  for (int c = 0; c < ci; ++c) {
    int init = 0;
    double init_e = 0.0;
    for (int o = 0; o < co; ++o) {
      const float* w = src + ((size_t)o * ci + c) * sp;
      double e = 0.0;
      for (int i = 0; i < sp; ++i) e += (double)w[i] * (double)w[i];
      if (e > init_e) {
        init = o;
        init_e = e;
      }
    }
    if (init_e == 0.0) continue;
    double nrm = std::sqrt(init_e);
    for (int i = 0; i < sp; ++i) dir[i] = (double)src[((size_t)init * ci + c) * sp + i] / nrm;
    for (int it = 0; it < 4; ++it) {
      for (int o = 0; o < co; ++o) {
        const float* w = src + ((size_t)o * ci + c) * sp;
        double s = 0.0;
        for (int i = 0; i < sp; ++i) s += (double)w[i] * dir[i];
        scales[o] = s;
      }
      double se = 0.0;
      for (int o = 0; o < co; ++o) se += scales[o] * scales[o];
      ENSURE(std::isfinite(se) && se > 0.0, "rank-one convolution factorization became degenerate");
      for (int i = 0; i < sp; ++i) {
        double s = 0.0;
        for (int o = 0; o < co; ++o) s += (double)src[((size_t)o * ci + c) * sp + i] * scales[o];
        dir[i] = s / se;
      }
      double n2 = 0.0;
      for (int i = 0; i < sp; ++i) n2 += dir[i] * dir[i];
      n2 = std::sqrt(n2);
      ENSURE(std::isfinite(n2) && n2 > 0.0, "rank-one convolution spatial factor became degenerate");
      for (int i = 0; i < sp; ++i) dir[i] /= n2;
    }
    for (int o = 0; o < co; ++o) {
      const float* w = src + ((size_t)o * ci + c) * sp;
      double s = 0.0;
      for (int i = 0; i < sp; ++i) s += (double)w[i] * dir[i];
      pw.v[(size_t)o * ci + c] = (float)s;
    }
    for (int i = 0; i < sp; ++i) dw.v[(size_t)c * sp + i] = (float)dir[i];
  }
  double max_src = 0, max_err = 0, src_e = 0, err_e = 0;
  for (int o = 0; o < co; ++o)
    for (int c = 0; c < ci; ++c) {
      float s = pw.v[(size_t)o * ci + c];
      for (int i = 0; i < sp; ++i) {
        float e = src[((size_t)o * ci + c) * sp + i];
        float a = s * dw.v[(size_t)c * sp + i];
        double err = (double)std::fabs(e - a);
        max_src = std::max(max_src, (double)std::fabs(e));
        max_err = std::max(max_err, err);
        src_e += (double)e * (double)e;
        err_e += err * err;
      }
    }
  double rel = src_e == 0.0 ? 0.0 : std::sqrt(err_e / src_e);
  double lim = max_src * 1e-5 + 1e-12;
  ENSURE(max_err <= lim && rel <= 1e-6, "fused convolution is not rank-one separable");
}

// fuse_intraclass_conv (src/cpu/model.rs:819-888): the k x 1 and 1 x k
// kernels are added into the centre column / row; biases are summed.
void fuse_intraclass(Tensor& sym, std::vector<float>& sb, const Tensor& vert, const std::vector<float>& vb,
                     const Tensor& hor, const std::vector<float>& hb) {
  int co = sym.shape[0], ci = sym.shape[1], k = sym.shape[2];
  int center = k / 2;
  for (int o = 0; o < co; ++o)
    for (int i = 0; i < ci; ++i) {
      size_t bo = ((size_t)o * ci + i) * k;
      size_t so = bo * k;
      const bool swap = fault(FAULT_INTRACLASS_ROW_COLUMN_SWAPPED);
      for (int r = 0; r < k; ++r) sym.v[so + (swap ? center * k + r : r * k + center)] += vert.v[bo + r];
      for (int c = 0; c < k; ++c) sym.v[so + (swap ? c * k + center : center * k + c)] += hor.v[bo + c];
    }
  for (int o = 0; o < co; ++o) {
    sb[o] += vb[o];
    sb[o] += hb[o];
  }
}

// RankOneConv2d (src/cpu/model.rs:165-219): depthwise k x k (no bias, pad
// k/2) then pointwise with bias.
struct RankOne {
  Conv dw, pw;
  Tensor forward(const Tensor& x) const { return pw.forward(dw.forward(x)); }
};

RankOne load_rank_one(const Weights& wt, const std::string& p, int ci, int co, int k) {
  Tensor W = wt.get(p + ".weight", {co, ci, k, k});
  RankOne r;
  r.dw.name = p + ".depthwise";
  r.pw.name = p + ".pointwise";
  factor_rank_one(W, ci, co, k, r.dw.W, r.pw.W);
  r.dw.groups = ci;
  for (int i = 0; i < 4; ++i) r.dw.pads[i] = k / 2;
  r.pw.b = wt.get(p + ".bias", {co}).v;
  return r;
}

// ---------------------------------------------------------------- necks

// RepLkFpn (src/cpu/model.rs:1197-1254) with ResidualSqueezeExcitation
// (:1107-1143) and DepthwiseSeparableConv (:1145-1195).
struct RepLkFpn {
  Conv in_conv[4];
  SE in_se[4];
  Conv dwc[4], pwc[4];
  SE dw_se[4];
  Tensor forward(const std::vector<Tensor>& st) const {
    std::vector<Tensor> fused;
    for (int i = 0; i < 4; ++i) {
      Tensor h = in_conv[i].forward(st[i]);
      Tensor g = in_se[i].gate(h);
      // Levels above the deepest add the upsampled level below before a
      // bf16 plan rounds them.
      const std::string name = "model.neck.fused." + std::to_string(i);
      fused.push_back(fault(FAULT_NECK_SE_PLAIN_GATE) ? mul_gate(h, g, name) : residual_mul_gate(h, g, name, i == 3));
      trace("fpn.insert" + std::to_string(i), fused.back());
    }
    const std::vector<Tensor> inserted = fused;
    for (int i = 2; i >= 0; --i)
      fused[i] = upsample_add(fused[i], fault(FAULT_TOPDOWN_NOT_CASCADED) ? inserted[i + 1] : fused[i + 1], 2,
                              "model.neck.fused." + std::to_string(i));
    std::vector<Tensor> feats;
    for (int i = 0; i < 4; ++i) {
      Tensor h = pwc[i].forward(dwc[i].forward(fused[i]));
      Tensor g = dw_se[i].gate(h);
      const std::string name = "model.neck.input_conv." + std::to_string(i) + ".out";
      feats.push_back(fault(FAULT_NECK_SE_PLAIN_GATE) ? mul_gate(h, g, name) : residual_mul_gate(h, g, name));
      trace("fpn.feature" + std::to_string(i), feats.back());
    }
    if (fault(FAULT_NECK_CONCAT_SHALLOW_FIRST)) return upsample_cat(feats, {1, 2, 4, 8});
    std::reverse(feats.begin(), feats.end());
    return upsample_cat(feats, {8, 4, 2, 1});
  }
};

RepLkFpn load_fpn(const Weights& wt, const int chans[4], int nc, int k) {
  RepLkFpn f;
  for (int i = 0; i < 4; ++i) {
    std::string p = "model.neck.insert_conv." + std::to_string(i);
    f.in_conv[i] = load_conv(wt, p + ".in_conv", chans[i], nc, 1, 1, 1, 1, {0, 0, 0, 0}, false, 1);
    f.in_se[i].reduce = load_conv(wt, p + ".squeeze_excitation_block.conv1", nc, nc / 4, 1, 1, 1, 1, {0, 0, 0, 0},
                                  true, 1);
    f.in_se[i].expand = load_conv(wt, p + ".squeeze_excitation_block.conv2", nc / 4, nc, 1, 1, 1, 1, {0, 0, 0, 0},
                                  true, 1);
    f.in_se[i].gate_act = fault(FAULT_NECK_SE_GATE_SIXTH) ? ACT_HSIG6 : ACT_HSIG5;
    std::string q = "model.neck.input_conv." + std::to_string(i);
    int pd = k / 2;
    f.dwc[i] = load_conv(wt, q + ".depthwise_convolution", nc, nc, k, k, 1, 1, {pd, pd, pd, pd}, true, nc);
    f.pwc[i] = load_conv(wt, q + ".pointwise_convolution", nc, nc / 4, 1, 1, 1, 1, {0, 0, 0, 0}, false, 1);
    f.dw_se[i].reduce = load_conv(wt, q + ".squeeze_excitation_module.conv1", nc / 4, nc / 16, 1, 1, 1, 1,
                                  {0, 0, 0, 0}, true, 1);
    f.dw_se[i].expand = load_conv(wt, q + ".squeeze_excitation_module.conv2", nc / 16, nc / 4, 1, 1, 1, 1,
                                  {0, 0, 0, 0}, true, 1);
    f.dw_se[i].gate_act = fault(FAULT_NECK_SE_GATE_SIXTH) ? ACT_HSIG6 : ACT_HSIG5;
  }
  return f;
}

// IntraclassBlock (src/cpu/model.rs:811-946).
struct Intraclass {
  Conv reduce, lng, mid, sht, fin;
  Tensor forward(const Tensor& x) const {
    Tensor r = reduce.forward(x);
    Tensor l7 = lng.forward(r);
    Tensor l5 = mid.forward(l7);
    Tensor l3 = sht.forward(l5);
    return add(x, fin.forward(l3, -1, false), fin.name);
  }
};

Conv load_fused_intraclass(const Weights& wt, const std::string& p, const std::string& ratio, int k) {
  Conv sym = load_conv(wt, p + ".symmetric_conv_long_" + ratio, 32, 32, k, k, 1, 1, {k / 2, k / 2, k / 2, k / 2},
                       true, 1);
  sym.name = p + (ratio == "longratio" ? ".long" : ratio == "midratio" ? ".mid" : ".short");
  Tensor vw = wt.get(p + ".vertical_long_to_small_conv_" + ratio + ".weight", {32, 32, k, 1});
  auto vb = wt.get(p + ".vertical_long_to_small_conv_" + ratio + ".bias", {32}).v;
  Tensor hw = wt.get(p + ".horizontal_small_to_long_conv_" + ratio + ".weight", {32, 32, 1, k});
  auto hb = wt.get(p + ".horizontal_small_to_long_conv_" + ratio + ".bias", {32}).v;
  fuse_intraclass(sym.W, sym.b, vw, vb, hw, hb);
  return sym;
}

// DetectorNeck, medium (src/cpu/model.rs:948-1067).
struct MediumNeck {
  Conv adjust[4];
  RankOne project[4], lateral[4];
  Conv pan[3];
  Intraclass intra[4];
  Tensor forward(const std::vector<Tensor>& st) const {
    std::vector<Tensor> adj;
    // Levels above the deepest add the upsampled level below before a bf16
    // plan rounds them.
    for (int i = 0; i < 4; ++i) adj.push_back(adjust[i].forward(st[i], -1, i == 3));
    std::vector<Tensor> td(4);
    td[3] = adj[3];
    for (int i = 2; i >= 0; --i)
      td[i] = upsample_add(adj[i], fault(FAULT_TOPDOWN_NOT_CASCADED) ? adj[i + 1] : td[i + 1], 2, adjust[i].name);
    std::vector<Tensor> bu, projected;
    for (int i = 0; i < 4; ++i) {
      Tensor p = project[i].forward(td[i]);
      projected.push_back(p);
      if (i > 0)
        p = add(p, pan[i - 1].forward(fault(FAULT_PAN_FROM_PROJECTION) ? projected[i - 1] : bu[i - 1], -1, false),
                pan[i - 1].name);
      bu.push_back(p);
      trace("neck.bottom_up" + std::to_string(i), p);
    }
    std::vector<Tensor> refined;
    for (int i = 0; i < 4; ++i) {
      Tensor l = lateral[i].forward(bu[i]);
      trace("neck.lateral" + std::to_string(i), l);
      refined.push_back(intra[i].forward(l));
      trace("neck.refined" + std::to_string(i), refined.back());
    }
    if (fault(FAULT_NECK_CONCAT_SHALLOW_FIRST)) return upsample_cat(refined, {1, 2, 4, 8});
    std::reverse(refined.begin(), refined.end());
    return upsample_cat(refined, {8, 4, 2, 1});
  }
};

MediumNeck load_medium_neck(const Weights& wt) {
  MediumNeck m;
  const int chans[4] = {128, 256, 512, 896};
  std::string n = "model.neck";
  for (int i = 0; i < 4; ++i) {
    std::string s = std::to_string(i);
    m.adjust[i] = load_conv(wt, n + ".input_channel_adjustment_convolution." + s, chans[i], 256, 1, 1, 1, 1,
                            {0, 0, 0, 0}, false, 1);
    m.project[i] = load_rank_one(wt, n + ".input_feature_projection_convolution." + s, 256, 64, 9);
    m.lateral[i] = load_rank_one(wt, n + ".path_aggregation_lateral_convolution." + s, 64, 64, 9);
    std::string p = n + ".intraclass_blocks." + s;
    m.intra[i].reduce = load_conv(wt, p + ".conv_reduce_channel", 64, 32, 1, 1, 1, 1, {0, 0, 0, 0}, true, 1);
    m.intra[i].lng = load_fused_intraclass(wt, p, "longratio", 7);
    m.intra[i].mid = load_fused_intraclass(wt, p, "midratio", 5);
    m.intra[i].sht = load_fused_intraclass(wt, p, "shortratio", 3);
    m.intra[i].fin = load_conv_bn(wt, p + ".conv_final", 32, 64, 1, 1, 1, 1, {0, 0, 0, 0}, true, 1, "norm", ACT_RELU);
  }
  for (int i = 0; i < 3; ++i)
    m.pan[i] = load_conv(wt, n + ".path_aggregation_head_convolution." + std::to_string(i), 64, 64, 3, 3, 2, 2,
                         {1, 1, 1, 1}, false, 1);
  return m;
}

// DetectorHead (src/cpu/model.rs:1419-1521): 3x3 (BN) ReLU, 2x2 s2 deconv
// (BN folded over output channels) ReLU, 2x2 s2 deconv to 1 + bias, sigmoid.
struct DetHead {
  Conv down;
  Tensor upW, finW;
  std::vector<float> upb, finb;
  Tensor forward(const Tensor& x) const {
    Tensor d = down.forward(x);
    trace("head.down", d);
    Tensor tmp;
    Tensor u = conv_transpose2x2(d, bf_weights(upW, tmp, "head.conv_up"), upb.data());
    act_in_place(u, ACT_RELU);
    trace("head.up", u);
    Tensor f = conv_transpose2x2(u, finW, finb.data());
    act_in_place(f, ACT_SIGMOID);
    return f;
  }
};

DetHead load_head(const Weights& wt, int nc) {
  DetHead h;
  int hid = nc / 4;
  h.down = load_conv_bn(wt, "head.conv_down", nc, hid, 3, 3, 1, 1, {1, 1, 1, 1}, false, 1, "norm", ACT_RELU);
  h.upW = wt.get("head.conv_up.convolution.weight", {hid, hid, 2, 2});
  h.upb = wt.get("head.conv_up.convolution.bias", {hid}).v;
  // fold_transpose_batch_norm (src/cpu/model.rs:1440-1477).
  Tensor g = wt.get("head.conv_up.norm.weight", {hid});
  Tensor be = wt.get("head.conv_up.norm.bias", {hid});
  Tensor mu = wt.get("head.conv_up.norm.running_mean", {hid});
  Tensor var = wt.get("head.conv_up.norm.running_var", {hid});
  for (int o = 0; o < hid; ++o) {
    float s = g.v[o] / std::sqrt(var.v[o] + 1e-5f);
    for (int i = 0; i < hid; ++i)
      for (int k = 0; k < 4; ++k)
        h.upW.v[(fault(FAULT_HEAD_BN_INPUT_AXIS) ? (size_t)o * hid + i : (size_t)i * hid + o) * 4 + k] *= s;
    h.upb[o] = (h.upb[o] - mu.v[o]) * s + be.v[o];
  }
  h.finW = wt.get("head.conv_final.weight", {hid, 1, 2, 2});
  h.finb = wt.get("head.conv_final.bias", {1}).v;
  return h;
}

// ---------------------------------------------------------------- models

struct Model {
  virtual ~Model() = default;
  virtual Tensor forward(const Tensor& x) const = 0;
  bool detector = true;
};

// Detector::load / forward (src/cpu/model.rs:1537-1625).
struct Detector : Model {
  int size = 2;
  Backbone bb;
  bool medium = false;
  RepLkFpn fpn;
  MediumNeck mneck;
  DetHead head;
  Tensor forward(const Tensor& x) const override {
    std::vector<Tensor> st = bb.forward(x);
    Tensor n = medium ? mneck.forward(st) : fpn.forward(st);
    trace("neck", n);
    return head.forward(n);
  }
};

// LightSVTR recognizer head (src/cpu/model.rs:1686-1875).
struct RecBlock {
  Tensor ln1w, ln1b, ln2w, ln2b, qkvW, qkvB, projW, projB, fc1W, fc1B, fc2W, fc2B;
  int hidden = 0, heads = 8;
  std::string p;  // module path head.encoder.svtr_block.<i>
  // The attention context, before its projection.
  Tensor attention(const Tensor& x) const {
    int B = x.shape[0], T = x.shape[1], hd = hidden / heads;
    Tensor qkv = linear(x, qkvW, &qkvB, ACT_NONE, false, p + ".self_attn.qkv");
    Tensor out({B, T, hidden});
    float scale = std::pow((float)(fault(FAULT_ATTENTION_SCALE_HIDDEN) ? hidden : hd), -0.5f);
    // Column of part (q, k, v) for head h, dimension d within a qkv row: the
    // row is viewed as [3, heads, hd] (src/cpu/model.rs:1706-1714).
    const bool head_major = fault(FAULT_QKV_HEAD_MAJOR);
    auto col = [&](int part, int h, int d) {
      return head_major ? (h * 3 + part) * hd + d : part * hidden + h * hd + d;
    };
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < heads; ++h) {
        std::vector<float> s(T);
        for (int t = 0; t < T; ++t) {
          const float* q = qkv.data() + ((size_t)b * T + t) * 3 * hidden;
          for (int u = 0; u < T; ++u) {
            const float* k = qkv.data() + ((size_t)b * T + u) * 3 * hidden;
            float acc = 0.0f;
            for (int dd = 0; dd < hd; ++dd) {
              const int d = g_reverse_sums ? hd - 1 - dd : dd;
              acc = std::fma(q[col(0, h, d)], k[col(1, h, d)], acc);
            }
            s[u] = std::fma(acc, scale, 0.0f);
          }
          softmax_row(s.data(), T);
          float* o = out.data() + ((size_t)b * T + t) * hidden + h * hd;
          for (int d = 0; d < hd; ++d) {
            float acc = 0.0f;
            for (int uu = 0; uu < T; ++uu) {
              const int u = g_reverse_sums ? T - 1 - uu : uu;
              acc = std::fma(s[u], qkv.v[((size_t)b * T + u) * 3 * hidden + col(2, h, d)], acc);
            }
            o[d] = acc;
          }
        }
      }
    return bf(out, p + ".self_attn");
  }
  // The projection and fc2 sums with their residuals are rounded once, after
  // the add, as a bf16 plan's epilogues do.
  Tensor forward(const Tensor& x) const {
    Tensor n1 = layer_norm(x, ln1w, ln1b, 1e-6f, p + ".layer_norm1");
    Tensor a = linear(attention(n1), projW, &projB, ACT_NONE, false, p + ".self_attn.projection", false);
    Tensor o = add(fault(FAULT_RECBLOCK_RESIDUAL_NORMED) ? n1 : x, a, p + ".self_attn.projection");
    Tensor h = linear(layer_norm(o, ln2w, ln2b, 1e-6f, p + ".layer_norm2"), fc1W, &fc1B, ACT_SILU, false,
                      p + ".mlp.fc1");
    Tensor m = linear(h, fc2W, &fc2B, ACT_NONE, false, p + ".mlp.fc2", false);
    return add(o, m, p + ".mlp.fc2");
  }
};

struct Recognizer : Model {
  int size = 2;
  Backbone bb;
  // tiny head (src/cpu/model.rs:1877-1936)
  Conv tconv1, tconv2;
  Tensor fc1W, fc1B, fc2W, fc2B;
  // LightSVTR
  Conv skip, reduce, local;
  RecBlock blocks[2];
  Tensor normW, normB, clsW, clsB;
  int hidden = 0;

  Tensor forward(const Tensor& x) const override {
    std::vector<Tensor> st = bb.forward(x);
    Tensor pooled = avg_pool_3x2(st.back(), "pool");  // [N, C, 1, T]
    trace("pool", pooled);
    int N = pooled.n(), C = pooled.c(), T = pooled.w();
    ENSURE(pooled.h() == 1, "recognizer pooling must produce height 1");
    if (size == 2) {
      Tensor h = tconv1.forward(pooled, fault(FAULT_TINY_HEAD_NO_HSWISH1) ? ACT_NONE : ACT_HSWISH);
      trace("tiny.conv1", h);
      h = tconv2.forward(h, ACT_HSWISH);
      trace("tiny.conv2", h);
      Tensor seq({N, T, C});
      for (int n = 0; n < N; ++n)
        for (int c = 0; c < C; ++c)
          for (int t = 0; t < T; ++t) seq.v[((size_t)n * T + t) * C + c] = h.v[((size_t)n * C + c) * T + t];
      return linear(linear(seq, fc1W, &fc1B, ACT_NONE, false, "head.fc1"), fc2W, &fc2B, ACT_NONE, true, "head.fc2");
    }
    // RecEncoder::forward (src/cpu/model.rs:1825-1842)
    Tensor res = skip.forward(pooled);
    trace("svtr.skip", res);
    Tensor h = reduce.forward(pooled);
    Tensor loc = local.forward(h, -1, false);
    h = add(h, loc, local.name);
    trace("svtr.hidden", h);
    int Hc = h.c();
    Tensor seq({N, T, Hc});
    for (int n = 0; n < N; ++n)
      for (int c = 0; c < Hc; ++c)
        for (int t = 0; t < T; ++t) seq.v[((size_t)n * T + t) * Hc + c] = h.v[((size_t)n * Hc + c) * T + t];
    for (size_t i = 0; i < 2; ++i) {
      seq = blocks[i].forward(seq);
      trace("svtr.block" + std::to_string(i), seq);
    }
    const bool skip_first = fault(FAULT_SVTR_SKIP_BEFORE_NORM);
    if (!skip_first) seq = layer_norm(seq, normW, normB, 1e-6f, "", false);
    for (int n = 0; n < N; ++n)
      for (int t = 0; t < T; ++t)
        for (int c = 0; c < Hc; ++c) {
          float& v = seq.v[((size_t)n * T + t) * Hc + c];
          v = v + res.v[((size_t)n * Hc + c) * T + t];
        }
    if (skip_first) seq = layer_norm(seq, normW, normB, 1e-6f, "", false);
    bf(seq, "head.encoder.norm");  // LayerNorm + skip, stored in bf16 by a bf16 plan
    trace("svtr.encoder", seq);
    return linear(seq, clsW, &clsB, ACT_NONE, true, "head.head");
  }
};

std::unique_ptr<Model> load_detector(const std::string& path, int size) {
  Weights wt = Weights::load(path);
  const size_t expected = size == 0 ? 350 : 271;
  ENSURE(wt.t.size() == expected, "detector has " + std::to_string(wt.t.size()) + " tensors; expected " +
                                      std::to_string(expected));
  auto d = std::make_unique<Detector>();
  d->size = size;
  int chans[4];
  int mid, out, nc;
  if (size == 0) {
    int c[4] = {128, 256, 512, 896};
    memcpy(chans, c, sizeof c);
    mid = 64, out = 128, nc = 256;
  } else if (size == 1) {
    int c[4] = {48, 96, 192, 384};
    memcpy(chans, c, sizeof c);
    mid = 24, out = 48, nc = 96;
  } else {
    int c[4] = {32, 48, 64, 160};
    memcpy(chans, c, sizeof c);
    mid = 16, out = 32, nc = 64;
  }
  d->bb = load_backbone(wt, mid, out, detector_stages(chans[0], chans[1], chans[2], chans[3]), true);
  if (size == 0) {
    d->medium = true;
    d->mneck = load_medium_neck(wt);
  } else {
    d->fpn = load_fpn(wt, chans, nc, size == 1 ? 7 : 5);
  }
  d->head = load_head(wt, nc);
  return d;
}

RecBlock load_rec_block(const Weights& wt, const std::string& p, int h, int mlp) {
  RecBlock b;
  b.p = p;
  b.hidden = h;
  b.ln1w = wt.get(p + ".layer_norm1.weight", {h});
  b.ln1b = wt.get(p + ".layer_norm1.bias", {h});
  b.qkvW = wt.get(p + ".self_attn.qkv.weight", {3 * h, h});
  b.qkvB = wt.get(p + ".self_attn.qkv.bias", {3 * h});
  b.projW = wt.get(p + ".self_attn.projection.weight", {h, h});
  b.projB = wt.get(p + ".self_attn.projection.bias", {h});
  b.ln2w = wt.get(p + ".layer_norm2.weight", {h});
  b.ln2b = wt.get(p + ".layer_norm2.bias", {h});
  b.fc1W = wt.get(p + ".mlp.fc1.weight", {mlp, h});
  b.fc1B = wt.get(p + ".mlp.fc1.bias", {mlp});
  b.fc2W = wt.get(p + ".mlp.fc2.weight", {h, mlp});
  b.fc2B = wt.get(p + ".mlp.fc2.bias", {h});
  return b;
}

std::unique_ptr<Model> load_recognizer(const std::string& path, int size) {
  Weights wt = Weights::load(path);
  const size_t expected = size == 0 ? 269 : size == 1 ? 250 : 150;
  ENSURE(wt.t.size() == expected, "recognizer has " + std::to_string(wt.t.size()) + " tensors; expected " +
                                      std::to_string(expected));
  auto r = std::make_unique<Recognizer>();
  r->detector = false;
  r->size = size;
  if (size == 2) {
    r->bb = load_backbone(wt, 24, 48, recognizer_stages(2), false);
    // Conv1dBn (src/cpu/model.rs:1877-1911): [O, I/g, k] folded then viewed
    // as [O, I/g, 1, k] with pads [0, k/2, 0, k/2].
    Tensor w1 = wt.get("head.conv1.weight", {160, 1, 5});
    w1.shape = {160, 1, 1, 5};
    std::vector<float> b1;
    fold_bn(w1, b1, wt, "head.norm1", 160);
    r->tconv1.name = "head.conv1";
    r->tconv1.W = w1;
    r->tconv1.b = b1;
    r->tconv1.groups = 160;
    r->tconv1.pads[1] = 2;
    r->tconv1.pads[3] = 2;
    Tensor w2 = wt.get("head.conv2.weight", {160, 160, 1});
    w2.shape = {160, 160, 1, 1};
    std::vector<float> b2;
    fold_bn(w2, b2, wt, "head.norm2", 160);
    r->tconv2.name = "head.conv2";
    r->tconv2.W = w2;
    r->tconv2.b = b2;
    r->fc1W = wt.get("head.fc1.weight", {80, 160});
    r->fc1B = wt.get("head.fc1.bias", {80});
    r->fc2W = wt.get("head.fc2.weight", {6906, 80});
    r->fc2B = wt.get("head.fc2.bias", {6906});
    return r;
  }
  int mid = size == 0 ? 64 : 48, out = size == 0 ? 128 : 96;
  int ci = size == 0 ? 768 : 384, h = size == 0 ? 192 : 120, mlp = size == 0 ? 768 : 240;
  r->hidden = h;
  r->bb = load_backbone(wt, mid, out, recognizer_stages(size), true);
  std::string e = "head.encoder";
  r->skip = load_conv_bn(wt, e + ".conv_block.0", ci, h, 1, 1, 1, 1, {0, 0, 0, 0}, false, 1, "normalization",
                         ACT_SILU);
  r->reduce = load_conv_bn(wt, e + ".conv_block.1", ci, h, 1, 1, 1, 1, {0, 0, 0, 0}, false, 1, "normalization",
                           ACT_SILU);
  r->local = load_conv_bn(wt, e + ".conv_block.2", h, h, 1, 7, 1, 1, {0, 3, 0, 3}, false, h, "normalization",
                          ACT_SILU);
  for (int i = 0; i < 2; ++i) r->blocks[i] = load_rec_block(wt, e + ".svtr_block." + std::to_string(i), h, mlp);
  r->normW = wt.get(e + ".norm.weight", {h});
  r->normB = wt.get(e + ".norm.bias", {h});
  r->clsW = wt.get("head.head.weight", {18710, h});
  r->clsB = wt.get("head.head.bias", {18710});
  return r;
}

// ---------------------------------------------------------------- preprocess

// normalized_bgr + scalar row kernel (src/preprocess.rs:78-123,
// src/preprocess/kernels.rs:94-170): quad-bilinear source point, clamped,
// bilinear RGB rounded to an integer, then v * (1/(255 std)) - mean/std.
// Columns at or beyond content_width stay zero.
void preprocess(const uint8_t* px, int sw, int sh, const float corners[8], int cw, int ch, int content_w,
                const float mean[3], const float stdv[3], float* out) {
  float scale[3], bias[3];
  for (int c = 0; c < 3; ++c) {
    scale[c] = 1.0f / (255.0f * stdv[c]);
    bias[c] = -mean[c] / stdv[c];
  }
  size_t plane = (size_t)ch * cw;
  std::fill(out, out + 3 * plane, 0.0f);
  float max_x = (float)(sw - 1), max_y = (float)(sh - 1);
#pragma omp parallel for schedule(static)
  for (int y = 0; y < ch; ++y) {
    float v = ((float)y + 0.5f) / (float)ch;
    float omv = 1.0f - v;
    for (int x = 0; x < content_w; ++x) {
      float u = ((float)x + 0.5f) / (float)content_w;
      float omu = 1.0f - u;
      float sx = std::clamp((corners[0] * omu + corners[2] * u) * omv + (corners[6] * omu + corners[4] * u) * v - 0.5f,
                            0.0f, max_x);
      float sy = std::clamp((corners[1] * omu + corners[3] * u) * omv + (corners[7] * omu + corners[5] * u) * v - 0.5f,
                            0.0f, max_y);
      int x0 = (int)std::floor(sx), y0 = (int)std::floor(sy);
      int x1 = std::min(x0 + 1, sw - 1), y1 = std::min(y0 + 1, sh - 1);
      float tx = sx - (float)x0, ty = sy - (float)y0;
      size_t o00 = ((size_t)y0 * sw + x0) * 3, o01 = ((size_t)y0 * sw + x1) * 3;
      size_t o10 = ((size_t)y1 * sw + x0) * 3, o11 = ((size_t)y1 * sw + x1) * 3;
      float rgb[3];
      for (int c = 0; c < 3; ++c) {
        float tl = px[o00 + c], tr = px[o01 + c], bl = px[o10 + c], br = px[o11 + c];
        float top = tl * (1.0f - tx) + tr * tx;
        float bot = bl * (1.0f - tx) + br * tx;
        rgb[c] = std::clamp(std::round(top * (1.0f - ty) + bot * ty), 0.0f, 255.0f);
      }
      // B, G, R planes.
      out[0 * plane + (size_t)y * cw + x] = rgb[2] * scale[0] + bias[0];
      out[1 * plane + (size_t)y * cw + x] = rgb[1] * scale[1] + bias[1];
      out[2 * plane + (size_t)y * cw + x] = rgb[0] * scale[2] + bias[2];
    }
  }
}

template <typename F>
int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return 1;
  }
}

}  // namespace

// ---------------------------------------------------------------- C API

extern "C" {

const char* oracle_last_error(void) { return g_error.c_str(); }

void oracle_set_threads(int threads) {
  if (threads > 0) omp_set_num_threads(threads);
}

// size: 0 medium, 1 small, 2 tiny (reference ModelSize order).
void* oracle_detector_load(const char* path, int size) {
  Model* m = nullptr;
  if (guarded([&] { m = load_detector(path, size).release(); })) return nullptr;
  return m;
}

void* oracle_recognizer_load(const char* path, int size) {
  Model* m = nullptr;
  if (guarded([&] { m = load_recognizer(path, size).release(); })) return nullptr;
  return m;
}

void oracle_model_free(void* m) { delete static_cast<Model*>(m); }

// Test hooks (see "test hooks" above).  A fault applies to models loaded and
// run while it is set; tracing keeps the tensors of the last forward.
int oracle_fault_count(void) { return FAULT_COUNT; }
void oracle_set_fault(int f) { g_fault = f; }
void oracle_set_bf16(int on) { g_bf16 = on != 0; }
void oracle_set_reverse_sums(int on) { g_reverse_sums = on != 0; }

// The emulation's rounding of n floats (tests pin it against a library
// bf16 conversion).
void oracle_round_bf16(const float* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = round_bf16(in[i]);
}

// The rounding points of the last forward run with the bf16 emulation on,
// one per line ("A <value>" or "W <layer>"), into `out` (NUL terminated, cut
// at `cap`); returns the bytes needed with the terminator.
long oracle_bf16_log(char* out, size_t cap) {
  std::string text;
  for (const std::string& r : g_bf16_log) text += r + "\n";
  if (out && cap) {
    const size_t k = std::min(cap - 1, text.size());
    memcpy(out, text.data(), k);
    out[k] = 0;
  }
  return (long)text.size() + 1;
}
void oracle_set_tracing(int on) {
  g_tracing = on != 0;
  g_trace.clear();
}

// Copies the traced tensor `name` into out (cap floats); returns its element
// count (0 if absent) and writes its shape (unused dims 0).
long oracle_trace_get(const char* name, float* out, size_t cap, int shape[4]) {
  auto it = g_trace.find(name);
  if (it == g_trace.end()) return 0;
  const Tensor& t = it->second;
  for (int i = 0; i < 4; ++i) shape[i] = i < (int)t.shape.size() ? t.shape[i] : 0;
  if (out && cap >= t.count()) memcpy(out, t.data(), t.count() * 4);
  return (long)t.count();
}

// Detector input: [N,3,H,W] with H,W % 32 == 0 -> [N,1,H,W].
// Recognizer input: [N,3,48,W] -> [N,T,V] (src/cpu/model.rs:1627-1646).
int oracle_forward(void* handle, const float* in, const int shape[4], float* out, size_t cap, int out_shape[4]) {
  return guarded([&] {
    Model* m = static_cast<Model*>(handle);
    ENSURE(shape[0] > 0, "input batch must not be empty");
    ENSURE(shape[1] == 3, "input must have three NCHW channels");
    ENSURE(shape[2] > 0 && shape[3] > 0, "input spatial dimensions must be positive");
    if (m->detector) {
      ENSURE(shape[2] % 32 == 0 && shape[3] % 32 == 0, "detector input height and width must be multiples of 32");
    } else {
      ENSURE(shape[2] == 48, "recognizer input height must be 48");
      ENSURE(shape[3] >= 5, "recognizer input width must be at least 5");
    }
    Tensor x({shape[0], shape[1], shape[2], shape[3]});
    memcpy(x.data(), in, x.count() * 4);
    g_bf16_log.clear();
    bf(x, "input");  // a bf16 plan stores its input in bf16
    Tensor y = m->forward(x);
    ENSURE(y.count() <= cap, "output buffer too small");
    memcpy(out, y.data(), y.count() * 4);
    for (int i = 0; i < 4; ++i) out_shape[i] = i < (int)y.shape.size() ? y.shape[i] : 0;
  });
}

int oracle_preprocess(const uint8_t* rgb, int sw, int sh, const float corners[8], int cw, int ch, int content_w,
                      int detector, float* out) {
  return guarded([&] {
    ENSURE(sw > 0 && sh > 0 && cw > 0 && ch > 0 && content_w > 0 && content_w <= cw, "preprocess geometry");
    const float dm[3] = {0.485f, 0.456f, 0.406f}, ds[3] = {0.229f, 0.224f, 0.225f};
    const float rm[3] = {0.5f, 0.5f, 0.5f}, rs[3] = {0.5f, 0.5f, 0.5f};
    preprocess(rgb, sw, sh, corners, cw, ch, content_w, detector ? dm : rm, detector ? ds : rs, out);
  });
}

// ---- single-operation entry points used by the known-answer tests.

float oracle_erf(float x) { return erf_as(x); }
float oracle_act(int act, float x) { return apply_act(act, x); }

int oracle_conv2d(const float* x, const int xs[4], const float* w, const int ws[4], const float* bias, int sh, int sw,
                  const int pads[4], int groups, int act, float* out, int out_shape[4]) {
  return guarded([&] {
    Tensor X({xs[0], xs[1], xs[2], xs[3]}), W({ws[0], ws[1], ws[2], ws[3]});
    memcpy(X.data(), x, X.count() * 4);
    memcpy(W.data(), w, W.count() * 4);
    Tensor y = conv2d(X, W, bias, sh, sw, pads, groups, act);
    memcpy(out, y.data(), y.count() * 4);
    for (int i = 0; i < 4; ++i) out_shape[i] = y.shape[i];
  });
}

int oracle_conv_transpose2x2(const float* x, const int xs[4], const float* w, const int ws[4], const float* bias,
                             float* out) {
  return guarded([&] {
    Tensor X({xs[0], xs[1], xs[2], xs[3]}), W({ws[0], ws[1], ws[2], ws[3]});
    memcpy(X.data(), x, X.count() * 4);
    memcpy(W.data(), w, W.count() * 4);
    Tensor y = conv_transpose2x2(X, W, bias);
    memcpy(out, y.data(), y.count() * 4);
  });
}

int oracle_linear(const float* x, long rows, int k, const float* w, int m, const float* bias, int act, int softmax,
                  float* out) {
  return guarded([&] {
    Tensor X({(int)rows, k}), W({m, k});
    memcpy(X.data(), x, X.count() * 4);
    memcpy(W.data(), w, W.count() * 4);
    Tensor B({m});
    if (bias) memcpy(B.data(), bias, (size_t)m * 4);
    Tensor y = linear(X, W, bias ? &B : nullptr, act, softmax != 0);
    memcpy(out, y.data(), y.count() * 4);
  });
}

void oracle_softmax(float* v, int n) { softmax_row(v, n); }
void oracle_layer_norm(float* v, const float* w, const float* b, int n, float eps) { layer_norm_row(v, w, b, n, eps); }
float oracle_residual_mul(float v, float g) { return residual_mul(v, g); }

int oracle_max_pool_same(const float* x, const int xs[4], float* out) {
  return guarded([&] {
    Tensor X({xs[0], xs[1], xs[2], xs[3]});
    memcpy(X.data(), x, X.count() * 4);
    Tensor y = max_pool_2x2_same(X);
    memcpy(out, y.data(), y.count() * 4);
  });
}

int oracle_avg_pool_3x2(const float* x, const int xs[4], float* out, int out_shape[4]) {
  return guarded([&] {
    Tensor X({xs[0], xs[1], xs[2], xs[3]});
    memcpy(X.data(), x, X.count() * 4);
    Tensor y = avg_pool_3x2(X);
    memcpy(out, y.data(), y.count() * 4);
    for (int i = 0; i < 4; ++i) out_shape[i] = y.shape[i];
  });
}

int oracle_upsample_add(float* feature, const int fs[4], const float* upper, const int us[4], int scale) {
  return guarded([&] {
    Tensor F({fs[0], fs[1], fs[2], fs[3]}), U({us[0], us[1], us[2], us[3]});
    memcpy(F.data(), feature, F.count() * 4);
    memcpy(U.data(), upper, U.count() * 4);
    Tensor y = upsample_add(F, U, scale);
    memcpy(feature, y.data(), y.count() * 4);
  });
}

// upsample_and_cat_nchw over `count` features with per-feature scales.
int oracle_upsample_cat(int count, const float* const* feats, const int* shapes /*count x 4*/, const int* scales,
                        float* out, int out_shape[4]) {
  return guarded([&] {
    std::vector<Tensor> fs;
    std::vector<int> sc;
    for (int i = 0; i < count; ++i) {
      Tensor t({shapes[4 * i], shapes[4 * i + 1], shapes[4 * i + 2], shapes[4 * i + 3]});
      memcpy(t.data(), feats[i], t.count() * 4);
      fs.push_back(std::move(t));
      sc.push_back(scales[i]);
    }
    Tensor y = upsample_cat(fs, sc);
    memcpy(out, y.data(), y.count() * 4);
    for (int i = 0; i < 4; ++i) out_shape[i] = y.shape[i];
  });
}

// Attention block core: qkv [B, T, 3h] -> context [B, T, h] (before the
// projection), as RecAttention::forward (src/cpu/model.rs:1703-1725).
int oracle_attention(const float* qkv, int B, int T, int hidden, int heads, float* out) {
  return guarded([&] {
    ENSURE(hidden % heads == 0, "hidden size must divide into heads");
    int hd = hidden / heads;
    float scale = std::pow((float)hd, -0.5f);
    std::vector<float> s(T);
    for (int bb = 0; bb < B; ++bb)
      for (int h = 0; h < heads; ++h)
        for (int t = 0; t < T; ++t) {
          const float* q = qkv + ((size_t)bb * T + t) * 3 * hidden + h * hd;
          for (int u = 0; u < T; ++u) {
            const float* k = qkv + ((size_t)bb * T + u) * 3 * hidden + hidden + h * hd;
            float acc = 0.0f;
            for (int d = 0; d < hd; ++d) acc = std::fma(q[d], k[d], acc);
            s[u] = std::fma(acc, scale, 0.0f);
          }
          softmax_row(s.data(), T);
          for (int d = 0; d < hd; ++d) {
            float acc = 0.0f;
            for (int u = 0; u < T; ++u)
              acc = std::fma(s[u], qkv[((size_t)bb * T + u) * 3 * hidden + 2 * hidden + h * hd + d], acc);
            out[((size_t)bb * T + t) * hidden + h * hd + d] = acc;
          }
        }
  });
}

int oracle_factor_rank_one(const float* w, int ci, int co, int k, float* dw, float* pw) {
  return guarded([&] {
    Tensor W({co, ci, k, k});
    memcpy(W.data(), w, W.count() * 4);
    Tensor D, P;
    factor_rank_one(W, ci, co, k, D, P);
    memcpy(dw, D.data(), D.count() * 4);
    memcpy(pw, P.data(), P.count() * 4);
  });
}

int oracle_fuse_intraclass(float* sym, float* sb, const float* vert, const float* vb, const float* hor,
                           const float* hb, int co, int ci, int k) {
  return guarded([&] {
    Tensor S({co, ci, k, k}), V({co, ci, k, 1}), H({co, ci, 1, k});
    memcpy(S.data(), sym, S.count() * 4);
    memcpy(V.data(), vert, V.count() * 4);
    memcpy(H.data(), hor, H.count() * 4);
    std::vector<float> b(sb, sb + co), vbv(vb, vb + co), hbv(hb, hb + co);
    fuse_intraclass(S, b, V, vbv, H, hbv);
    memcpy(sym, S.data(), S.count() * 4);
    memcpy(sb, b.data(), (size_t)co * 4);
  });
}

}  // extern "C"
