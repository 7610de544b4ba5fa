// Plan builders: PP-OCRv6 detectors (tiny/small/medium) and recognizers
// (tiny/small/medium) as lists of gfx950 kernel launches over NHWC views of
// one activation arena.
//
// The architecture follows the reference CPU model (src/cpu/model.rs); the
// load-time transforms are the reference's: BatchNorm folding
// (src/cpu/model.rs:371-407, :1440-1477), rank-one factorisation of the
// medium neck's 9x9 convs (:221-369) and intraclass kernel fusion
// (:819-888).  Where the reference's WGSL path runs several kernels, this
// plan fuses: SE gates are applied while the next 1x1 conv gathers its input
// and again on its residual, FPN top-down adds and upsample-concats happen in
// the producers' epilogues, and the DB head's two transposed convs and the
// sigmoid run as one kernel.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "runtime.h"

namespace ppocr {
namespace {

constexpr size_t NOW = SIZE_MAX;

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

uint16_t to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);  // NaN stays NaN
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// f rounded to bf16 (nearest even), as a float.
float bf16_value(float f) {
  const uint32_t u = (uint32_t)to_bf16(f) << 16;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

struct ConvW {
  size_t w = NOW, b = NOW;  // byte offsets into the weight blob
  int ldw = 0;
  int ci = 0, ci_pad = 0, co = 0, kh = 1, kw = 1, sh = 1, sw = 1, pt = 0, pl = 0, pb = 0, pr = 0;
};

struct DwW {
  size_t w = NOW, b = NOW, tab = NOW;  // tab: matrix-core tap fragments (bf16 plans)
  int c = 0, kh = 1, kw = 1, sh = 1, sw = 1, pt = 0, pl = 0, pb = 0, pr = 0;
};

struct SeW {
  size_t w1 = NOW, b1 = NOW, w2 = NOW, b2 = NOW;
  int c = 0, cr = 0, act = ACT_HSIG6;
};

struct Epi {
  int act = ACT_NONE;
  const View* in_gate = nullptr;
  const View* res = nullptr;
  const View* res_gate = nullptr;
  const View* up = nullptr;
  int up_s = 2;
  int rep = 1;
  const View* dst = nullptr;  // write into this (pre-allocated) view
};

struct BlockSpec {
  int ci, co, sh, sw;
  bool se;
};

class Builder {
 public:
  Builder(const SafeTensors& st, Plan& plan, int dt) : st_(st), plan_(plan), dt_(dt) { plan_.dt = dt; }

  int dt() const { return dt_; }

  // ------------------------------------------------------------ weights
  HostTensor get(const std::string& name, const std::vector<int>& shape) { return st_.get(name, shape); }

  // s = gamma / sqrt(var + 1e-5); W' = W s per output channel;
  // b' = (b - mean) s + beta (src/cpu/model.rs:371-407).  With `transposed`
  // the weight is IOHW [ci][co][k] and the scale applies along its second
  // axis (fold_transpose_batch_norm, src/cpu/model.rs:1440-1477).
  void fold_bn(std::vector<float>& W, std::vector<float>& b, const std::string& norm, int co, bool transposed = false,
               int ci = 0) {
    HostTensor g = get(norm + ".weight", {co}), be = get(norm + ".bias", {co});
    HostTensor mu = get(norm + ".running_mean", {co}), var = get(norm + ".running_var", {co});
    if (b.empty()) b.assign(co, 0.0f);
    if (!transposed) {
      size_t row = W.size() / co;
      for (int o = 0; o < co; ++o) {
        float s = g.v[o] / std::sqrt(var.v[o] + 1e-5f);
        for (size_t i = 0; i < row; ++i) W[o * row + i] *= s;
        b[o] = (b[o] - mu.v[o]) * s + be.v[o];
      }
    } else {
      size_t k = W.size() / ((size_t)ci * co);
      for (int o = 0; o < co; ++o) {
        float s = g.v[o] / std::sqrt(var.v[o] + 1e-5f);
        for (int i = 0; i < ci; ++i)
          for (size_t t = 0; t < k; ++t) W[((size_t)i * co + o) * k + t] *= s;
        b[o] = (b[o] - mu.v[o]) * s + be.v[o];
      }
    }
  }

  // Appends fp32 values to the weight blob (256-byte aligned); returns the
  // byte offset.
  size_t put(const std::vector<float>& v) {
    size_t off = round_up(plan_.weights.size(), 256);
    plan_.weights.resize(off + v.size() * 4, 0);
    memcpy(plan_.weights.data() + off, v.data(), v.size() * 4);
    return off;
  }

  // Appends values in the activation storage type (matrix-core operands).
  size_t put_act(const std::vector<float>& v) {
    if (dt_ == DT_F32) return put(v);
    size_t off = round_up(plan_.weights.size(), 256);
    plan_.weights.resize(off + v.size() * 2, 0);
    uint16_t* dst = reinterpret_cast<uint16_t*>(plan_.weights.data() + off);
    for (size_t i = 0; i < v.size(); ++i) dst[i] = to_bf16(v[i]);
    return off;
  }

  // OIHW [co][ci][kh][kw] -> [co][k = (ky*kw + kx)*ci_pad + c]; the padded
  // input channels get zero weights.
  ConvW pack_conv(const std::vector<float>& W, const std::vector<float>& b, int ci, int co, int kh, int kw, int sh,
                  int sw, std::vector<int> pads, int ci_pad = 0) {
    ConvW c;
    c.ci = ci;
    c.ci_pad = ci_pad ? ci_pad : ci;
    c.co = co;
    c.kh = kh, c.kw = kw, c.sh = sh, c.sw = sw;
    c.pt = pads[0], c.pl = pads[1], c.pb = pads[2], c.pr = pads[3];
    if (c.ci_pad % 4) raise(PPOCR_ERR_INVALID_MODEL, "conv input channels must be padded to a multiple of 4");
    size_t K = (size_t)kh * kw * c.ci_pad;
    c.ldw = (int)K;
    std::vector<float> packed((size_t)co * K, 0.0f);
    for (int o = 0; o < co; ++o)
      for (int i = 0; i < ci; ++i)
        for (int ky = 0; ky < kh; ++ky)
          for (int kx = 0; kx < kw; ++kx)
            packed[(size_t)o * K + (size_t)(ky * kw + kx) * c.ci_pad + i] = W[(((size_t)o * ci + i) * kh + ky) * kw + kx];
    c.w = put_act(packed);
    if (!b.empty()) c.b = put(b);
    return c;
  }

  // [c][kh*kw] -> [kh*kw][c].
  DwW pack_dw(const std::vector<float>& W, const std::vector<float>& b, int c, int kh, int kw, int sh, int sw,
              std::vector<int> pads) {
    DwW d;
    d.c = c, d.kh = kh, d.kw = kw, d.sh = sh, d.sw = sw;
    d.pt = pads[0], d.pl = pads[1], d.pb = pads[2], d.pr = pads[3];
    std::vector<float> packed((size_t)kh * kw * c);
    for (int ch = 0; ch < c; ++ch)
      for (int t = 0; t < kh * kw; ++t) packed[(size_t)t * c + ch] = W[(size_t)ch * kh * kw + t];
    // bf16 plans take 5x5 and wider taps in bf16 (the matrix-core form's
    // operand type) on every kernel: the vector-ALU kernels, which run the
    // maps too small for the matrix cores and the gate-residual layers, read
    // the same bf16-valued taps in fp32.
    if (dt_ == DT_BF16 && kh >= 5 && kw >= 5)
      for (float& v : packed) v = bf16_value(v);
    d.w = put(packed);
    if (!b.empty()) d.b = put(b);
    if (depthwise_uses_mfma(kh, kw, sh, sw, dt_, 16, c)) {
      std::vector<uint16_t> tab(depthwise_mfma_table_size(c, kh));
      depthwise_mfma_table(W.data(), c, kh, tab.data());
      size_t off = round_up(plan_.weights.size(), 256);
      plan_.weights.resize(off + tab.size() * 2, 0);
      memcpy(plan_.weights.data() + off, tab.data(), tab.size() * 2);
      d.tab = off;
    }
    return d;
  }

  // Conv2d::load (src/cpu/model.rs:89-107) and Conv2d::load_bn (:110-131).
  ConvW conv_w(const std::string& p, int ci, int co, int kh, int kw, int sh, int sw, std::vector<int> pads, bool bias,
               const std::string& norm = "", int ci_pad = 0) {
    std::string wname = norm.empty() ? p + ".weight" : p + ".convolution.weight";
    std::string bname = norm.empty() ? p + ".bias" : p + ".convolution.bias";
    std::vector<float> W = get(wname, {co, ci, kh, kw}).v;
    std::vector<float> b;
    if (bias) b = get(bname, {co}).v;
    if (!norm.empty()) fold_bn(W, b, p + "." + norm, co);
    return pack_conv(W, b, ci, co, kh, kw, sh, sw, pads, ci_pad);
  }

  DwW dw_w(const std::string& p, int c, int kh, int kw, int sh, int sw, std::vector<int> pads, bool bias,
           const std::string& norm = "") {
    std::string wname = norm.empty() ? p + ".weight" : p + ".convolution.weight";
    std::vector<float> W = get(wname, {c, 1, kh, kw}).v;
    std::vector<float> b;
    if (bias) b = get(p + ".bias", {c}).v;
    if (!norm.empty()) fold_bn(W, b, p + "." + norm, c);
    return pack_dw(W, b, c, kh, kw, sh, sw, pads);
  }

  SeW se_w(const std::string& reduce, const std::string& expand, int c, int cr, int act) {
    SeW s;
    s.c = c, s.cr = cr, s.act = act;
    s.w1 = put(get(reduce + ".weight", {cr, c, 1, 1}).v);
    s.b1 = put(get(reduce + ".bias", {cr}).v);
    s.w2 = put(get(expand + ".weight", {c, cr, 1, 1}).v);
    s.b2 = put(get(expand + ".bias", {c}).v);
    return s;
  }

  // Linear::new (src/cpu/backend.rs:1244-1280): weight [out][in] + bias.
  ConvW linear_w(const std::string& p, int fin, int fout) {
    std::vector<float> W = get(p + ".weight", {fout, fin}).v;
    std::vector<float> b = get(p + ".bias", {fout}).v;
    return pack_conv(W, b, fin, fout, 1, 1, 1, 1, {0, 0, 0, 0});
  }

  // ------------------------------------------------------------ values
  // A new buffer in the activation storage type (or `dt` when given).
  View alloc(int n, int h, int w, int c, const std::string& name, int dt = -1, int ps = 0) {
    View v;
    v.n = n, v.h = h, v.w = w, v.c = c, v.ps = ps ? ps : c;
    v.dt = dt < 0 ? dt_ : dt;
    Buffer b;
    b.bytes = (size_t)n * h * w * v.ps * dtype_size(v.dt);
    b.name = name;
    b.dt = v.dt;
    plan_.bufs.push_back(b);
    v.buf = (int)plan_.bufs.size() - 1;
    return v;
  }

  static View slice(View v, int c0, int c) {
    v.off += c0;
    v.c = c;
    return v;
  }

  void add_op(Op op) {
    int idx = (int)plan_.ops.size();
    for (int b : op.reads) touch(b, idx);
    for (int b : op.writes) touch(b, idx);
    plan_.ops.push_back(std::move(op));
  }

  void touch(int b, int idx) {
    Buffer& buf = plan_.bufs[b];
    if (buf.first < 0 || idx < buf.first) buf.first = idx;
    buf.last = std::max(buf.last, idx);
  }

  // ------------------------------------------------------------ ops
  // Name of the kernel instance launch_conv will run for `base` reading view
  // x with weights at blob offset wo.  The pointers are stood in for by
  // their offsets, which decide their alignment: arena buffers and weight
  // offsets are 256-byte aligned.  `terms`: the epilogue inputs the launch
  // will pass (kTermRes, kTermResGate, kTermUp, kTermCtc), stood in for by
  // non-null aligned values.
  static constexpr unsigned kTermRes = 1, kTermResGate = 2, kTermUp = 4, kTermCtc = 8;
  static std::string conv_kernel(const ConvParams& base, const View& x, size_t wo, bool gated, unsigned terms = 0) {
    return conv_kernel_name(stand_in(base, x, wo, gated, terms));
  }
  // `base` with its pointers stood in for as above.
  static ConvParams stand_in(const ConvParams& base, const View& x, size_t wo, bool gated, unsigned terms) {
    ConvParams probe = base;
    probe.in = reinterpret_cast<const void*>((uintptr_t)(x.off * dtype_size(x.dt)));
    probe.wt = reinterpret_cast<const void*>((uintptr_t)wo);
    probe.in_gate = gated ? reinterpret_cast<const float*>((uintptr_t)16) : nullptr;
    const uintptr_t nonnull = 256;
    if (terms & kTermRes) probe.res = reinterpret_cast<const void*>(nonnull);
    if (terms & kTermResGate) probe.res_gate = reinterpret_cast<const float*>(nonnull);
    if (terms & kTermUp) probe.up = reinterpret_cast<const void*>(nonnull);
    if (terms & kTermCtc) probe.ctc_part = reinterpret_cast<float*>(nonnull);
    return probe;
  }

  // Channel sums of a layer's output left by the depthwise or conv kernel
  // that writes it, for the squeeze-excitation that reads it next: [N][P][C]
  // fp32.
  struct SePartial {
    View part;
    int P = 0;
  };

  // A conv op not yet added: its op and the function that fills its launch
  // parameters (for merging independent layers into one launch).
  struct Deferred {
    Op op;
    std::function<ConvParams(const Exec&)> fill;
    ConvParams shape;  // its parameters with stand-in pointers
  };

  // With sp, the conv also leaves the channel sums of its output in *sp
  // where its kernel can (sp->P = 0 otherwise).  With `gated`, a bf16 layer
  // with an SE input gate returns there the x * g tensor its gate pass stores.
  // With `defer`, the op is returned there instead of added.
  View conv(const View& x, const ConvW& w, const Epi& e, const std::string& name, SePartial* sp = nullptr,
            View* gated = nullptr, Deferred* defer = nullptr) {
    if (x.c != w.ci_pad) raise(PPOCR_ERR_INVALID_MODEL, name + ": input has " + std::to_string(x.c) + " channels");
    const int Ho = (x.h + w.pt + w.pb - w.kh) / w.sh + 1;
    const int Wo = (x.w + w.pl + w.pr - w.kw) / w.sw + 1;
    const int oh = Ho * e.rep, ow = Wo * e.rep;
    if ((e.res || e.res_gate || e.up || e.rep != 1) && w.co % 4)
      raise(PPOCR_ERR_INVALID_MODEL, name + ": fused epilogue terms need a multiple of 4 output channels");
    View out;
    if (e.dst) {
      out = *e.dst;
      if (out.h != oh || out.w != ow || out.c != w.co || out.n != x.n)
        raise(PPOCR_ERR_INVALID_MODEL, name + ": destination shape mismatch");
    } else {
      out = alloc(x.n, oh, ow, w.co, name);
    }
    if (out.dt != x.dt && (e.res || e.up || e.rep != 1))
      raise(PPOCR_ERR_INVALID_MODEL, name + ": mixed-type epilogue is limited to plain stores");
    View in = x;
    View res = e.res ? *e.res : View();
    View rg = e.res_gate ? *e.res_gate : View();
    View ig = e.in_gate ? *e.in_gate : View();
    View up = e.up ? *e.up : View();
    bool has_res = e.res, has_rg = e.res_gate, has_ig = e.in_gate, has_up = e.up;
    // bf16 layers with an SE input gate: a separate pass writes x * g
    // (rounded to bf16, the value the gather would form) and the GEMM runs
    // ungated on the direct kernel; applying the gate per operand fragment
    // would cost more vector instructions than the bf16 MFMAs take.
    const bool prescale = has_ig && x.dt == DT_BF16;
    View xs;
    if (prescale) xs = alloc(x.n, x.h, x.w, x.c, name + ".gated");
    if (gated) *gated = xs;
    const View& a_src = prescale ? xs : x;
    ConvParams base{};
    base.N = x.n, base.H = x.h, base.W = x.w, base.C = x.c, base.in_ps = a_src.ps;
    base.Ho = Ho, base.Wo = Wo, base.Co = w.co, base.out_ps = out.ps;
    base.out_f32 = out.dt == DT_F32 && x.dt != DT_F32;
    base.ldw = w.ldw;
    base.kh = w.kh, base.kw = w.kw, base.sh = w.sh, base.sw = w.sw, base.pt = w.pt, base.pl = w.pl;
    base.act = e.act;
    base.res_ps = has_res ? res.ps : 0;
    base.up_s = e.up_s;
    base.up_ps = has_up ? up.ps : 0;
    base.rep = e.rep;
    base.out_h = oh, base.out_w = ow;
    base.dt = x.dt;
    size_t wo = w.w, bo = w.b;
    // Split-K workspace [splits][M][Co] fp32, live for this op only.
    const int splits = conv_split_k(x.n * Ho * Wo, w.co, w.kh * w.kw * x.c, x.dt);
    View ws;
    if (splits > 1) ws = alloc(1, splits, x.n * Ho * Wo, w.co, name + ".split_k", DT_F32);
    base.splits = splits;
    const unsigned terms = (has_res ? kTermRes : 0u) | (has_rg ? kTermResGate : 0u) | (has_up ? kTermUp : 0u);
    View part;
    bool has_part = false;
    if (sp) {
      sp->P = 0;
      const int P = conv_se_blocks(stand_in(base, a_src, wo, has_ig && !prescale, terms));
      if (P > 0) {
        part = alloc(1, P, 1, w.co, name + ".se_partial", DT_F32);
        has_part = true;
        sp->part = part;
        sp->P = P;
      }
    }
    Op op;
    op.name = name;
    if (dt_ == DT_BF16) op.bf16_weights = {name};
    op.kernel = conv_kernel(base, a_src, wo, has_ig && !prescale, terms);
    if (prescale) op.kernel += "+gate_pass";
    if (splits > 1) op.kernel += "+split_k" + std::to_string(splits);
    op.bound = 1;
    const double es = (double)dtype_size(x.dt);
    double M = (double)x.n * Ho * Wo;
    double K = (double)w.kh * w.kw * w.ci;
    double cols = w.co;
    op.flops = 2.0 * M * cols * K;
    op.bytes = es * ((double)x.pixels() * w.ci + K * cols + (has_res ? M * w.co : 0.0) +
                     (has_up ? (double)up.pixels() * w.co : 0.0)) +
               (double)dtype_size(out.dt) * (double)out.pixels() * w.co;
    op.reads = {x.buf};
    if (has_res) op.reads.push_back(res.buf);
    if (has_rg) op.reads.push_back(rg.buf);
    if (has_ig) op.reads.push_back(ig.buf);
    if (has_up) op.reads.push_back(up.buf);
    op.writes = {out.buf};
    if (splits > 1) op.writes.push_back(ws.buf);
    if (prescale) op.writes.push_back(xs.buf);
    if (has_part) op.writes.push_back(part.buf);
    auto fill = [=](const Exec& ex) {
      ConvParams p = base;
      p.in = prescale ? ex.ptr(xs) : ex.ptr(in);
      p.in_gate = has_ig && !prescale ? ex.fptr(ig) : nullptr;
      p.out = ex.ptr(out);
      p.wt = ex.wv(wo);
      p.bias = ex.w(bo);
      p.res = has_res ? ex.ptr(res) : nullptr;
      p.res_gate = has_rg ? ex.fptr(rg) : nullptr;
      p.up = has_up ? ex.ptr(up) : nullptr;
      p.split_ws = splits > 1 ? ex.fptr(ws) : nullptr;
      p.se_part = has_part ? ex.fptr(part) : nullptr;
      return p;
    };
    op.launch = [=](const Exec& ex, hipStream_t s) {
      if (prescale)
        launch_scale_channels(ex.ptr(in), in.n, in.h * in.w, in.c, in.ps, ex.fptr(ig), ex.ptr(xs), in.dt, s);
      launch_conv(fill(ex), s);
    };
    if (defer) {
      ConvParams shape = stand_in(base, a_src, wo, has_ig && !prescale, terms);
      shape.splits = splits;
      shape.se_part = has_part ? reinterpret_cast<float*>((uintptr_t)256) : nullptr;
      *defer = Deferred{std::move(op), fill, shape};
    } else {
      add_op(std::move(op));
    }
    return out;
  }

  // Independent conv layers (the levels of a neck), each set of them that
  // can share a launch (conv_multi_supported) as one op, the others one op
  // each; a set is named after `name` with its first layer's index.
  std::vector<View> conv_levels(const std::vector<const View*>& xs, const std::vector<ConvW>& ws, const Epi& e,
                                const std::vector<std::string>& names, const std::string& name,
                                std::vector<SePartial>* sps = nullptr) {
    const int n = (int)xs.size();
    std::vector<View> outs(n);
    std::vector<Deferred> d(n);
    for (int i = 0; i < n; ++i)
      outs[i] = conv(*xs[i], ws[i], e, names[i], sps ? &(*sps)[i] : nullptr, nullptr, &d[i]);
    // Greedy sets in layer order: a layer joins the first set it can share a
    // launch with.
    std::vector<std::vector<int>> sets;
    for (int i = 0; i < n; ++i) {
      bool placed = false;
      for (auto& set : sets) {
        if ((int)set.size() >= kConvMultiMax) continue;
        std::vector<ConvParams> shapes;
        for (int j : set) shapes.push_back(d[j].shape);
        shapes.push_back(d[i].shape);
        if (conv_multi_supported(shapes.data(), (int)shapes.size())) {
          set.push_back(i);
          placed = true;
          break;
        }
      }
      if (!placed) sets.push_back({i});
    }
    for (auto& set : sets) {
      if (set.size() == 1) {
        add_op(std::move(d[set[0]].op));
        continue;
      }
      std::vector<Deferred*> members;
      for (int j : set) members.push_back(&d[j]);
      add_multi(members, sets.size() == 1 ? name : name + "." + std::to_string(set[0]));
    }
    return outs;
  }

  void add_multi(const std::vector<Deferred*>& d, const std::string& name) {
    Op op;
    op.name = name;
    op.kernel = d[0]->op.kernel + "x" + std::to_string(d.size());
    op.bound = 1;
    std::vector<std::function<ConvParams(const Exec&)>> fills;
    for (Deferred* qp : d) {
      Deferred& q = *qp;
      op.flops += q.op.flops;
      op.bytes += q.op.bytes;
      op.reads.insert(op.reads.end(), q.op.reads.begin(), q.op.reads.end());
      op.writes.insert(op.writes.end(), q.op.writes.begin(), q.op.writes.end());
      op.bf16_weights.insert(op.bf16_weights.end(), q.op.bf16_weights.begin(), q.op.bf16_weights.end());
      fills.push_back(q.fill);
    }
    op.launch = [fills](const Exec& ex, hipStream_t s) {
      ConvMulti m{};
      m.count = (int)fills.size();
      for (int i = 0; i < m.count; ++i) m.p[i] = fills[i](ex);
      launch_conv_multi(m, s);
    };
    add_op(std::move(op));
  }

  // Depthwise conv.  With se_cr > 0 a squeeze-excitation of reduction width
  // se_cr reads the output next; when the kernel can, and the gate is not
  // small enough for its one-kernel form (or sums_always), it also leaves
  // the gate's channel sums in *sp (sp->P = 0 otherwise).
  // The FPN gate-residual x = h + h * g (+ up2(upper)) applied as the
  // depthwise conv's input prologue: `x` passed to depthwise() is h, and
  // `out` (when set) receives x itself for the layers that read it next.
  struct GateResidual {
    View gate;
    const View* upper = nullptr;
    const View* out = nullptr;
    std::string name;  // of the value x, rounded to the storage type also where it is not stored
  };

  View depthwise(const View& x, const DwW& w, int act, const View* res, const std::string& name, int se_cr = 0,
                 SePartial* sp = nullptr, const GateResidual* gr = nullptr, bool sums_always = false) {
    if (x.c != w.c) raise(PPOCR_ERR_INVALID_MODEL, name + ": channel mismatch");
    if (gr && (res || se_cr || !depthwise_gate_residual_supported(w.kh, w.kw, w.sh, w.sw) || w.pt != w.kh / 2 ||
               w.pl != w.kw / 2 || (gr->upper && (x.h != 2 * gr->upper->h || x.w != 2 * gr->upper->w))))
      raise(PPOCR_ERR_INVALID_MODEL, name + ": gate-residual prologue needs a plain same-size 5x5, 7x7 or 9x9 layer");
    int Ho = (x.h + w.pt + w.pb - w.kh) / w.sh + 1;
    int Wo = (x.w + w.pl + w.pr - w.kw) / w.sw + 1;
    View out = alloc(x.n, Ho, Wo, w.c, name);
    DwParams base{};
    base.N = x.n, base.H = x.h, base.W = x.w, base.C = x.c, base.in_ps = x.ps;
    base.Ho = Ho, base.Wo = Wo, base.out_ps = out.ps;
    base.kh = w.kh, base.kw = w.kw, base.sh = w.sh, base.sw = w.sw, base.pt = w.pt, base.pl = w.pl;
    base.act = act;
    base.dt = x.dt;
    View part;
    bool has_part = false;
    if (sp) {
      sp->P = 0;
      SeParams se{};
      se.N = x.n, se.HW = Ho * Wo, se.C = w.c, se.Cr = se_cr, se.dt = x.dt;
      const int P = depthwise_se_blocks(base);
      if (se_cr > 0 && P > 0 && (sums_always || !se_fused(se))) {
        part = alloc(x.n, P, 1, w.c, name + ".se_partial", DT_F32);
        has_part = true;
        sp->part = part;
        sp->P = P;
      }
    }
    View in = x;
    View r = res ? *res : View();
    bool has_res = res;
    base.res_ps = has_res ? r.ps : 0;
    size_t wo = w.w, bo = w.b, to = w.tab;
    Op op;
    op.name = name;
    if (dt_ == DT_BF16 && w.kh >= 5 && w.kw >= 5) op.bf16_weights = {name};
    if (dt_ == DT_BF16 && gr) {
      op.rounds = {name, gr->name};
      op.rounds_set = true;
    }
    op.kernel = depthwise_kernel_name(w.kh, w.kw, w.sh, w.sw, Ho, x.dt, w.tab != NOW && x.ps % 8 == 0, w.c,
                                      x.ps % 8 == 0 && out.ps % 8 == 0 && (!res || res->ps % 8 == 0));
    op.flops = 2.0 * out.pixels() * w.c * w.kh * w.kw;
    op.bytes = (double)dtype_size(x.dt) * ((double)x.pixels() * w.c + (double)out.pixels() * w.c * (has_res ? 2 : 1)) +
               4.0 * w.kh * w.kw * w.c;
    // 5x5 and larger taps on the VALU kernels do more fp32 FMAs per byte than
    // the vector ALU can retire at the HBM rate; the matrix-core form is
    // HBM-bound again.
    if (w.kh * w.kw >= 25 && op.kernel.rfind("depthwise_mfma", 0) != 0) op.bound = 2;
    op.reads = {x.buf};
    if (has_res) op.reads.push_back(r.buf);
    op.writes = {out.buf};
    if (has_part) op.writes.push_back(part.buf);
    const bool has_gr = gr, has_up = gr && gr->upper, has_grout = gr && gr->out;
    const View grg = gr ? gr->gate : View(), gru = has_up ? *gr->upper : View(), gro = has_grout ? *gr->out : View();
    if (has_gr) {
      op.kernel += "+gate_residual";
      op.reads.push_back(grg.buf);
      if (has_up) op.reads.push_back(gru.buf);
      if (has_grout) op.writes.push_back(gro.buf);
      const double px = (double)x.pixels() * w.c * dtype_size(x.dt);
      op.bytes += (has_up ? px / 4 : 0.0) + (has_grout ? px : 0.0);
      base.gr_up_ps = has_up ? gru.ps : 0;
      base.gr_out_ps = has_grout ? gro.ps : 0;
    }
    op.launch = [=](const Exec& ex, hipStream_t s) {
      DwParams p = base;
      p.in = ex.ptr(in);
      p.out = ex.ptr(out);
      p.wt = ex.w(wo);
      p.bias = ex.w(bo);
      p.res = has_res ? ex.ptr(r) : nullptr;
      p.se_part = has_part ? ex.fptr(part) : nullptr;
      p.wtab = ex.w(to);
      if (has_gr) {
        p.gr_gate = ex.fptr(grg);
        p.gr_up = has_up ? ex.ptr(gru) : nullptr;
        p.gr_out = has_grout ? ex.ptr(gro) : nullptr;
      }
      launch_depthwise(p, s);
    };
    add_op(std::move(op));
    return out;
  }

  // The LCNet pointwise pair as one fused op (pair_gemm.hip): channel_conv1
  // (GELU) and channel_conv2 with the hidden tile on chip; `gate` is the SE
  // gate of x (or null) and `residual` adds the gated x.  With `dw` (no
  // gate), x is the input of the block's 3x3 depthwise token conv `dw`,
  // which the op computes per tile instead of reading its stored output.
  // With se_sums and se (no gate view), the kernel forms x's SE gate itself
  // from the channel sums the token conv left (pair_se_fold_supported).
  View pointwise_pair(const View& x, const ConvW& w1, const ConvW& w2, const View* gate, bool residual,
                      const std::string& name, const DwW* dw = nullptr, const SePartial* se_sums = nullptr,
                      const SeW* se = nullptr) {
    if (dw && (gate || se_sums || dw->kh != 3 || dw->kw != 3 || dw->c != x.c))
      raise(PPOCR_ERR_INVALID_MODEL, name + ": depthwise prologue needs an ungated 3x3 depthwise");
    const bool fold = se_sums && se;
    if (fold && (gate || !pair_se_fold_supported(x.n, x.c, w1.co, se->cr, se_sums->P) || se->c != x.c))
      raise(PPOCR_ERR_INVALID_MODEL, name + ": SE gate in the pair prologue is not supported for this shape");
    const int h = dw ? (x.h + dw->pt + dw->pb - 3) / dw->sh + 1 : x.h;
    const int w = dw ? (x.w + dw->pl + dw->pr - 3) / dw->sw + 1 : x.w;
    if (x.c != w1.ci_pad || w2.ci_pad != w1.co || w1.kh * w1.kw * w2.kh * w2.kw != 1)
      raise(PPOCR_ERR_INVALID_MODEL, name + ": pointwise pair shapes do not chain");
    if (residual && w2.co != x.c) raise(PPOCR_ERR_INVALID_MODEL, name + ": residual needs equal channel counts");
    View out = alloc(x.n, h, w, w2.co, name);
    View in = x;
    View g = gate ? *gate : View();
    const bool has_gate = gate || fold;
    const View part = fold ? se_sums->part : View();
    const SeW sw = fold ? *se : SeW();
    PairParams base{};
    if (fold) base.se_P = se_sums->P, base.se_Cr = sw.cr, base.se_act = sw.act;
    base.in_ps = x.ps;
    base.HW = h * w;
    base.M = x.n * h * w;
    base.C = x.c, base.H2 = w1.co, base.Co = w2.co;
    base.ldw1 = w1.ldw, base.ldw2 = w2.ldw;
    base.residual = residual;
    base.out_ps = out.ps;
    if (dw) {
      base.dw_ps = x.ps, base.dw_h = x.h, base.dw_w = x.w, base.dw_wo = w;
      base.dw_sh = dw->sh, base.dw_sw = dw->sw, base.dw_pt = dw->pt, base.dw_pl = dw->pl;
    }
    const size_t w1o = w1.w, b1o = w1.b, w2o = w2.w, b2o = w2.b;
    const size_t dwo = dw ? dw->w : NOW, dbo = dw ? dw->b : NOW;
    const bool has_dw = dw;
    Op op;
    op.name = name;
    op.kernel = std::string("pointwise_pair") + (has_gate ? "<gate>" : has_dw ? "<dw3x3>" : "") + (fold ? "+se" : "");
    op.bound = 1;
    const double M = (double)base.M;
    op.flops = 2.0 * M * ((double)x.c * w1.co + (double)w1.co * w2.co + (has_dw ? 9.0 * x.c : 0.0));
    op.bytes = 4.0 * ((double)x.pixels() * x.c + (double)x.c * w1.co + (double)w1.co * w2.co + M * w2.co +
                      (has_dw ? 10.0 * x.c : 0.0));
    if (fold) {
      op.flops += 2.0 * 2.0 * x.c * sw.cr;
      op.bytes += 4.0 * ((double)se_sums->P * x.c + 2.0 * x.c * sw.cr);
    }
    op.reads = {x.buf};
    if (gate) op.reads.push_back(g.buf);
    if (fold) op.reads.push_back(part.buf);
    op.writes = {out.buf};
    op.launch = [=](const Exec& ex, hipStream_t s) {
      PairParams p = base;
      p.in = has_dw ? nullptr : ex.fptr(in);
      p.dw_in = has_dw ? ex.fptr(in) : nullptr;
      p.dw_wt = ex.w(dwo);
      p.dw_b = ex.w(dbo);
      p.gate = has_gate && !fold ? ex.fptr(g) : nullptr;
      if (fold) {
        p.se_part = ex.fptr(part);
        p.se_w1 = ex.w(sw.w1);
        p.se_b1 = ex.w(sw.b1);
        p.se_w2 = ex.w(sw.w2);
        p.se_b2 = ex.w(sw.b2);
      }
      p.w1 = ex.w(w1o);
      p.b1 = ex.w(b1o);
      p.w2 = ex.w(w2o);
      p.b2 = ex.w(b2o);
      p.out = ex.fptr(out);
      launch_pointwise_pair(p, s);
    };
    add_op(std::move(op));
    return out;
  }

  // bf16 plans: an LCNet block's pointwise pair x -> conv1 (GELU) -> conv2
  // (+ residual) in one launch (pair_bf16_supported shapes), `gate` the SE
  // gate of x or null.  It rounds where the unfused layers would (x * g,
  // the GELU output, the result) and writes only the result, named as
  // channel_conv2's output would be.
  View pointwise_pair_bf16(const View& x, const ConvW& w1, const ConvW& w2, const View* gate, bool residual,
                           const std::string& p) {
    if (x.dt != DT_BF16 || x.c != w1.ci_pad || w2.ci_pad != w1.co || w1.kh * w1.kw * w2.kh * w2.kw != 1 ||
        !pair_bf16_supported(x.c, w1.co, w2.co) || (residual && w2.co != x.c))
      raise(PPOCR_ERR_INVALID_MODEL, p + ": bf16 pointwise pair shapes do not chain");
    View out = alloc(x.n, x.h, x.w, w2.co, p + "2");
    PairBf16Params base{};
    base.in_ps = x.ps;
    base.HW = x.h * x.w;
    base.M = x.n * x.h * x.w;
    base.C = x.c;
    base.ldw1 = w1.ldw, base.ldw2 = w2.ldw;
    base.residual = residual;
    base.out_ps = out.ps;
    const bool has_gate = gate;
    const View in = x;
    const View g = gate ? *gate : View();
    const size_t w1o = w1.w, b1o = w1.b, w2o = w2.w, b2o = w2.b;
    Op op;
    op.name = p;
    // Stand-in pointers (offsets, 16-byte aligned like the real ones) pick the instance name.
    PairBf16Params probe = base;
    probe.gate = has_gate ? reinterpret_cast<const float*>((uintptr_t)256) : nullptr;
    op.kernel = pair_bf16_kernel_name(probe);
    op.bound = 1;
    const double M = (double)base.M, C = x.c, H = w1.co;
    op.flops = 2.0 * M * (C * H + H * w2.co);
    op.bytes = 2.0 * (M * C + C * H + H * w2.co + M * w2.co) + (has_gate ? 4.0 * x.n * C : 0.0);
    op.rounds = {p + "1", p + "2"};
    if (has_gate) op.rounds.push_back(p + "1.gated");
    op.rounds_set = true;
    op.bf16_weights = {p + "1", p + "2"};
    op.reads = {x.buf};
    if (has_gate) op.reads.push_back(g.buf);
    op.writes = {out.buf};
    op.launch = [=](const Exec& ex, hipStream_t s) {
      PairBf16Params q = base;
      q.in = ex.ptr(in);
      q.gate = has_gate ? ex.fptr(g) : nullptr;
      q.w1 = ex.wv(w1o);
      q.b1 = ex.w(b1o);
      q.w2 = ex.wv(w2o);
      q.b2 = ex.w(b2o);
      q.out = ex.ptr(out);
      launch_pair_bf16(q, s);
    };
    add_op(std::move(op));
    return out;
  }

  // Squeeze-excitation gate [N,1,1,C] (fp32) of x (src/cpu/model.rs:456-493,
  // :1069-1105).
  // With sp->P > 0 the channel sums come from the kernel that wrote x.
  View se(const View& x, const SeW& w, const std::string& name, const SePartial* sp = nullptr) {
    int HW = x.h * x.w;
    const bool given = sp && sp->P > 0;
    int P = given ? sp->P : std::max(1, std::min(HW / 64, std::max(1, 1024 / x.n)));
    SeParams base{};
    base.N = x.n, base.HW = HW, base.C = x.c, base.in_ps = x.ps, base.P = P, base.Cr = w.cr, base.gate_act = w.act;
    base.dt = x.dt;
    // Small gates run in one kernel without the partial and hidden arrays.
    const bool fused = !given && se_fused(base);
    View part, hid;
    if (given) {
      part = sp->part;
      hid = alloc(x.n, 1, 1, (int)round_up(w.cr, 4), name + ".hidden", DT_F32);
    } else if (!fused) {
      part = alloc(x.n, P, 1, x.c, name + ".partial", DT_F32);
      hid = alloc(x.n, 1, 1, (int)round_up(w.cr, 4), name + ".hidden", DT_F32);
    }
    View gate = alloc(x.n, 1, 1, x.c, name, DT_F32);
    View in = x;
    SeW ww = w;
    Op op;
    op.name = name;
    op.kernel = fused ? "se_fused" : given ? "se_gate+sums" : "se_gate";
    op.flops = 2.0 * x.n * ((double)HW * x.c + 2.0 * x.c * w.cr);
    op.bytes = (given ? 4.0 * x.n * P * x.c : (double)dtype_size(x.dt) * x.pixels() * x.c) +
               4.0 * (2.0 * x.c * w.cr + x.n * x.c);
    op.reads = {given ? part.buf : x.buf};
    op.writes = {gate.buf};
    if (given)
      op.writes.push_back(hid.buf);
    else if (!fused)
      op.writes.insert(op.writes.end(), {part.buf, hid.buf});
    op.launch = [=](const Exec& ex, hipStream_t s) {
      SeParams p = base;
      p.in = ex.ptr(in);
      p.partial = fused ? nullptr : ex.fptr(part);
      p.w1 = ex.w(ww.w1);
      p.b1 = ex.w(ww.b1);
      p.w2 = ex.w(ww.w2);
      p.b2 = ex.w(ww.b2);
      p.hidden = fused ? nullptr : ex.fptr(hid);
      p.gate = ex.fptr(gate);
      if (given)
        launch_se_from_partials(p, s);
      else
        launch_se(p, s);
    };
    add_op(std::move(op));
    return gate;
  }

  // The gates of several maps, each with the channel sums its producing conv
  // left: one launch where every gate takes the one-workgroup path with the
  // same kernel, otherwise one se() op per map.
  std::vector<View> se_levels(const std::vector<View>& xs, const std::vector<SeW>& ws, const std::string& name,
                              const std::vector<SePartial>& sps) {
    const int count = (int)xs.size();
    bool batch = count >= 2 && count <= kSeMultiMax;
    int kind = -1;
    std::vector<SeParams> ps(count);
    for (int i = 0; batch && i < count; ++i) {
      const View& x = xs[i];
      SeParams& b = ps[i];
      b = SeParams{};
      b.N = x.n, b.HW = x.h * x.w, b.C = x.c, b.in_ps = x.ps, b.P = sps[i].P, b.Cr = ws[i].cr;
      b.gate_act = ws[i].act, b.dt = x.dt;
      const int k = sps[i].P > 0 ? se_multi_kind(b) : 0;
      batch = k != 0 && (kind < 0 || k == kind) && x.n == xs[0].n;
      kind = k;
    }
    std::vector<View> gates(count);
    if (!batch) {
      for (int i = 0; i < count; ++i) gates[i] = se(xs[i], ws[i], name + "." + std::to_string(i), &sps[i]);
      return gates;
    }
    std::vector<View> parts(count);
    std::vector<SeW> wv = ws;
    Op op;
    op.name = name;
    op.kernel = "se_gates+sums";
    op.flops = op.bytes = 0.0;
    for (int i = 0; i < count; ++i) {
      const View& x = xs[i];
      gates[i] = alloc(x.n, 1, 1, x.c, name + "." + std::to_string(i), DT_F32);
      parts[i] = sps[i].part;
      op.flops += 2.0 * x.n * ((double)x.h * x.w * x.c + 2.0 * x.c * ws[i].cr);
      op.bytes += 4.0 * x.n * sps[i].P * x.c + 4.0 * (2.0 * x.c * ws[i].cr + x.n * x.c);
      op.reads.push_back(parts[i].buf);
      op.writes.push_back(gates[i].buf);
    }
    op.launch = [=](const Exec& ex, hipStream_t s) {
      SeMulti m{};
      m.count = count;
      for (int i = 0; i < count; ++i) {
        SeParams p = ps[i];
        p.partial = ex.fptr(parts[i]);
        p.w1 = ex.w(wv[i].w1);
        p.b1 = ex.w(wv[i].b1);
        p.w2 = ex.w(wv[i].w2);
        p.b2 = ex.w(wv[i].b2);
        p.gate = ex.fptr(gates[i]);
        m.p[i] = p;
      }
      launch_se_multi(m, s);
    };
    add_op(std::move(op));
    return gates;
  }

  // x_i + x_i*g_i written replicated (rep_i) into dst_i for several maps of
  // the same image count and storage type, in one launch; level i's value is
  // named names[i].
  void gate_residual_levels(const std::vector<View>& xs, const std::vector<View>& gs, const std::vector<View>& dsts,
                            const std::vector<int>& reps, const std::string& name,
                            const std::vector<std::string>& names) {
    const int count = (int)xs.size();
    Op op;
    op.name = name;
    if (dt_ == DT_BF16) {
      op.rounds = names;
      op.rounds_set = true;
    }
    op.kernel = "gate_residual";
    op.bytes = 0.0;
    for (int i = 0; i < count; ++i) {
      op.bytes += (double)dtype_size(xs[i].dt) * xs[i].pixels() * xs[i].c * (1 + reps[i] * reps[i]);
      op.reads.push_back(xs[i].buf);
      op.reads.push_back(gs[i].buf);
      op.writes.push_back(dsts[i].buf);
    }
    std::vector<View> in = xs, gate = gs, out = dsts;
    std::vector<int> rep = reps;
    const int n = xs[0].n, dt = xs[0].dt;
    op.launch = [=](const Exec& ex, hipStream_t s) {
      GateResidualMulti m{};
      m.count = count, m.N = n, m.dt = dt;
      for (int i = 0; i < count; ++i)
        m.part[i] = GateResidualPart{ex.ptr(in[i]), in[i].h,          in[i].w, in[i].c, in[i].ps,
                                     ex.fptr(gate[i]), ex.ptr(out[i]), out[i].ps, rep[i]};
      launch_gate_residual_multi(m, s);
    };
    add_op(std::move(op));
  }

  // x + x*g [+ up2(upper)], written (optionally replicated) into dst.
  void gate_residual(const View& x, const View& g, const View* upper, const View& dst, int rep,
                     const std::string& name) {
    View in = x, gate = g, out = dst;
    View up = upper ? *upper : View();
    bool has_up = upper;
    Op op;
    op.name = name;
    op.kernel = "gate_residual";
    op.bytes = (double)dtype_size(x.dt) *
               ((double)x.pixels() * x.c * (1 + rep * rep) + (has_up ? (double)up.pixels() * x.c : 0.0));
    op.reads = {x.buf, g.buf};
    if (has_up) op.reads.push_back(up.buf);
    op.writes = {dst.buf};
    op.launch = [=](const Exec& ex, hipStream_t s) {
      launch_gate_residual(ex.ptr(in), in.n, in.h, in.w, in.c, in.ps, ex.fptr(gate), has_up ? ex.ptr(up) : nullptr,
                           has_up ? up.ps : 0, ex.ptr(out), out.ps, rep, in.dt, s);
    };
    add_op(std::move(op));
  }

  void maxpool_same(const View& x, const View& dst, const std::string& name) {
    View in = x, out = dst;
    Op op;
    op.name = name;
    op.kernel = "maxpool_same";
    op.exact = true;
    op.bytes = 2.0 * dtype_size(x.dt) * x.pixels() * x.c;
    op.reads = {x.buf};
    op.writes = {dst.buf};
    op.launch = [=](const Exec& ex, hipStream_t s) {
      launch_maxpool_same(ex.ptr(in), in.n, in.h, in.w, in.c, in.ps, ex.ptr(out), out.ps, in.dt, s);
    };
    add_op(std::move(op));
  }

  View avgpool32(const View& x, const std::string& name) {
    int Ho = (x.h - 3) / 3 + 1, Wo = (x.w - 2) / 2 + 1;
    View out = alloc(x.n, Ho, Wo, x.c, name);
    View in = x;
    Op op;
    op.name = name;
    op.kernel = "avgpool";
    op.bytes = (double)dtype_size(x.dt) * ((double)x.pixels() * x.c + (double)out.pixels() * x.c);
    op.reads = {x.buf};
    op.writes = {out.buf};
    op.launch = [=](const Exec& ex, hipStream_t s) {
      launch_avgpool32(ex.ptr(in), in.n, in.h, in.w, in.c, in.ps, ex.ptr(out), out.h, out.w, in.dt, s);
    };
    add_op(std::move(op));
    return out;
  }

  View layer_norm(const View& x, const std::string& p, const View* res, const std::string& name) {
    int C = x.c;
    size_t wo = put(get(p + ".weight", {C}).v), bo = put(get(p + ".bias", {C}).v);
    View out = alloc(x.n, x.h, x.w, C, name);
    View in = x;
    View r = res ? *res : View();
    bool has_res = res;
    Op op;
    op.name = name;
    op.kernel = "layer_norm";
    op.bytes = (double)dtype_size(x.dt) * x.pixels() * C * (has_res ? 3 : 2) + 8.0 * C;
    op.reads = {x.buf};
    if (has_res) op.reads.push_back(r.buf);
    op.writes = {out.buf};
    op.launch = [=](const Exec& ex, hipStream_t s) {
      launch_layer_norm(ex.ptr(in), (int)in.pixels(), C, ex.w(wo), ex.w(bo), 1e-6f, has_res ? ex.ptr(r) : nullptr,
                        ex.ptr(out), in.dt, s);
    };
    add_op(std::move(op));
    return out;
  }

  // LayerNorm `p` (eps 1e-6) of x fused into the linear layer w that reads
  // it (pair_gemm.hip), with activation act.
  View ln_linear(const View& x, const std::string& p, const ConvW& w, int act, const std::string& name) {
    const int C = x.c;
    if (w.ci_pad != C || w.kh * w.kw != 1) raise(PPOCR_ERR_INVALID_MODEL, name + ": linear input mismatch");
    const size_t lwo = put(get(p + ".weight", {C}).v), lbo = put(get(p + ".bias", {C}).v);
    View out = alloc(x.n, x.h, x.w, w.co, name);
    View in = x;
    LnLinearParams base{};
    base.in_ps = x.ps;
    base.M = (int)x.pixels();
    base.K = C, base.N = w.co;
    base.eps = 1e-6f;
    base.ldw = w.ldw;
    base.act = act;
    base.out_ps = out.ps;
    const size_t wo = w.w, bo = w.b;
    Op op;
    op.name = name;
    op.kernel = "ln_linear";
    op.bound = 1;
    const double M = (double)x.pixels();
    op.flops = 2.0 * M * C * w.co;
    op.bytes = 4.0 * (M * C + (double)C * w.co + M * w.co) + 8.0 * C;
    op.reads = {x.buf};
    op.writes = {out.buf};
    op.launch = [=](const Exec& ex, hipStream_t s) {
      LnLinearParams q = base;
      q.in = ex.fptr(in);
      q.ln_w = ex.w(lwo);
      q.ln_b = ex.w(lbo);
      q.w = ex.w(wo);
      q.b = ex.w(bo);
      q.out = ex.fptr(out);
      launch_ln_linear(q, s);
    };
    add_op(std::move(op));
    return out;
  }

  View attention(const View& qkv, int hidden, int heads, const std::string& name) {
    View out = alloc(qkv.n, qkv.h, qkv.w, hidden, name);
    View in = qkv;
    int T = qkv.h * qkv.w;
    if (hidden % heads || attention_head_tile(hidden / heads) == 0)
      raise(PPOCR_ERR_INVALID_MODEL, name + ": head dimension must divide the hidden size and be at most 32");
    Op op;
    op.name = name;
    op.kernel = "attention";
    op.flops = 2.0 * qkv.n * heads * (double)T * T * (hidden / heads) * 2.0;
    op.bytes = (double)dtype_size(qkv.dt) * ((double)qkv.pixels() * 3 * hidden + (double)out.pixels() * hidden);
    op.reads = {qkv.buf};
    op.writes = {out.buf};
    op.launch = [=](const Exec& ex, hipStream_t s) {
      launch_attention(ex.ptr(in), in.n, T, hidden, heads, ex.ptr(out), in.dt, s);
    };
    add_op(std::move(op));
    return out;
  }

  void softmax(const View& x, const std::string& name) {
    if (x.dt != DT_F32) raise(PPOCR_ERR_INVALID_MODEL, name + ": softmax runs on fp32 rows");
    View io = x;
    Op op;
    op.name = name;
    op.kernel = "softmax";
    op.bytes = 8.0 * x.pixels() * x.c;
    op.reads = {x.buf};
    op.writes = {x.buf};
    op.launch = [=](const Exec& ex, hipStream_t s) { launch_softmax_rows(ex.fptr(io), (long)io.pixels(), io.c, s); };
    add_op(std::move(op));
  }

  // Classifier fused with the per-step half of greedy CTC decoding: for each
  // time step, the argmax class (ties -> last index) and its softmax
  // probability, the two values src/ocr.rs:800-853 takes from each row of
  // probabilities.  The logits are reduced inside the GEMM epilogue and never
  // stored.  Output [N, 1, T, 2] fp32: (class index, probability).
  View greedy_classifier(const View& x, const ConvW& w, const std::string& name) {
    if (x.c != w.ci_pad || w.kh != 1 || w.kw != 1 || x.h != 1)
      raise(PPOCR_ERR_INVALID_MODEL, name + ": greedy classifier takes [N, 1, T, C] rows");
    if (w.b == NOW) raise(PPOCR_ERR_INVALID_MODEL, name + ": classifier needs a bias");
    const int M = x.n * x.w;
    const int bn = conv_tile_cols(M, w.co, x.dt);
    const int tiles = (w.co + bn - 1) / bn;
    if ((size_t)3 * tiles * M > (size_t)INT32_MAX) raise(PPOCR_ERR_INVALID_INPUT, name + ": batch too large");
    View part = alloc(1, 1, 1, 3 * tiles * M, name + ".partials", DT_F32);
    View out = alloc(x.n, 1, x.w, 2, "output", DT_F32);
    ConvParams base{};
    base.N = x.n, base.H = 1, base.W = x.w, base.C = x.c, base.in_ps = x.ps;
    base.Ho = 1, base.Wo = x.w, base.Co = w.co, base.out_ps = 0;
    base.ldw = w.ldw;
    base.kh = base.kw = base.sh = base.sw = 1;
    base.act = ACT_NONE;
    base.up_s = 2;
    base.rep = 1;
    base.out_h = 1, base.out_w = x.w;
    base.dt = x.dt;
    const View in = x;
    const size_t wo = w.w, bo = w.b;
    const double es = (double)dtype_size(x.dt), part_bytes = 12.0 * tiles * M;
    Op op;
    op.name = name;
    op.kernel = conv_kernel(base, x, wo, false, kTermCtc);
    op.bound = 1;
    op.flops = 2.0 * M * w.co * w.ci;
    op.bytes = es * ((double)M * w.ci + (double)w.ci * w.co) + 4.0 * w.co + part_bytes;
    op.reads = {x.buf};
    op.writes = {part.buf};
    op.launch = [=](const Exec& ex, hipStream_t s) {
      ConvParams p = base;
      p.in = ex.ptr(in);
      p.out = nullptr;
      p.wt = ex.wv(wo);
      p.bias = ex.w(bo);
      p.ctc_part = ex.fptr(part);
      launch_conv(p, s);
    };
    add_op(std::move(op));
    Op merge;
    merge.name = name + ".ctc_merge";
    merge.kernel = "ctc_merge";
    merge.bytes = part_bytes + 8.0 * M;
    merge.reads = {part.buf};
    merge.writes = {out.buf};
    merge.launch = [=](const Exec& ex, hipStream_t s) { launch_ctc_merge(ex.fptr(part), M, tiles, ex.fptr(out), s); };
    add_op(std::move(merge));
    return out;
  }

  // fp32 NCHW staging buffer -> NHWC with 4 channels in the activation type.
  View input(const size_t nchw[4]) {
    int n = (int)nchw[0], h = (int)nchw[2], w = (int)nchw[3];
    View st = alloc(n, 3, h, w, "input.nchw", DT_F32);
    plan_.staging = st.buf;
    View x = alloc(n, h, w, 4, "input");
    Op op;
    op.name = "input";
    op.kernel = "nchw_to_nhwc";
    op.bytes = (12.0 + 4.0 * dtype_size(x.dt)) * n * h * w;
    op.reads = {st.buf};
    op.writes = {x.buf};
    op.launch = [=](const Exec& ex, hipStream_t s) {
      launch_nchw_to_nhwc4(ex.fptr(st), ex.ptr(x), n, h, w, x.dt, s);
    };
    add_op(std::move(op));
    plan_.input = x;
    return x;
  }

  Plan& plan() { return plan_; }

 private:
  const SafeTensors& st_;
  Plan& plan_;
  int dt_;
};

// ------------------------------------------------------------------ backbone

// LcNetBlock (src/cpu/model.rs:509-603).
// Whether an LCNet block's pointwise pair runs fused (pair_gemm.hip): fp32,
// channel counts in multiples of 16, and at most 64 input channels.  Wider
// pairs measured slower fused than as two GEMMs (pairs up to 192 channels
// fused: small detector at batch 1 0.87x, small recognizer at batch 1 0.74x):
// a workgroup owns 32 pixels, so the deep stages' few hundred pixels give a
// few workgroups where the two GEMMs split K over the whole GPU, and every
// workgroup streams both weight matrices from L2.
bool pair_fusion_pays(const View& t, int ci, int co, int dt) {
  (void)t;
  return ci <= 64 && pointwise_pair_supported(ci, 2 * ci, co, dt);
}

View lcnet_block(Builder& B, const View& x, const std::string& p, BlockSpec s) {
  bool residual = s.ci == s.co && s.sh == 1 && s.sw == 1;
  DwW tw = residual ? B.dw_w(p + ".token_conv", s.ci, 3, 3, s.sh, s.sw, {1, 1, 1, 1}, true)
                    : B.dw_w(p + ".token_conv", s.ci, 3, 3, s.sh, s.sw, {1, 1, 1, 1}, false, "normalization");
  bool has_se = s.se;
  ConvW c1 = B.conv_w(p + ".channel_conv1", s.ci, 2 * s.ci, 1, 1, 1, 1, {0, 0, 0, 0}, false, "normalization");
  ConvW c2 = B.conv_w(p + ".channel_conv2", 2 * s.ci, s.co, 1, 1, 1, 1, {0, 0, 0, 0}, false, "normalization");
  // Without SE the token conv's output feeds only the pair: the pair
  // computes it per tile (src/cpu/backend.rs:697-816).
  if (!has_se && pair_fusion_pays(x, s.ci, s.co, B.dt()))
    return B.pointwise_pair(x, c1, c2, nullptr, residual, p + ".channel_conv", &tw);
  // A single image's fused pair forms the SE gate in its own prologue from
  // the token conv's channel sums (no gate launch) where the sums are few.
  const bool pays = pair_fusion_pays(x, s.ci, s.co, B.dt());
  const bool fold = has_se && pays && x.n == 1;
  Builder::SePartial sums;
  View t = B.depthwise(x, tw, ACT_NONE, nullptr, p + ".token_conv", has_se ? s.ci / 4 : 0, &sums, nullptr, fold);
  View gate;
  SeW sw;
  if (has_se) {
    std::string q = p + ".token_squeeze_excitation.convolutions";
    sw = B.se_w(q + ".0", q + ".2", s.ci, s.ci / 4, ACT_HSIG6);
    if (fold && sums.P > 0 && pair_se_fold_supported(t.n, s.ci, 2 * s.ci, s.ci / 4, sums.P))
      return B.pointwise_pair(t, c1, c2, nullptr, residual, p + ".channel_conv", nullptr, &sums, &sw);
    gate = B.se(t, sw, p + ".se", &sums);
  }
  if (pays) return B.pointwise_pair(t, c1, c2, has_se ? &gate : nullptr, residual, p + ".channel_conv");
  if (B.dt() == DT_BF16 && pair_bf16_supported(s.ci, 2 * s.ci, s.co))
    return B.pointwise_pair_bf16(t, c1, c2, has_se ? &gate : nullptr, residual, p + ".channel_conv");
  Epi e1;
  e1.act = ACT_GELU;
  if (has_se) e1.in_gate = &gate;
  View gated;
  View h = B.conv(t, c1, e1, p + ".channel_conv1", nullptr, &gated);
  Epi e2;
  if (residual) {
    // The residual is the post-SE tensor: in a bf16 plan the stored
    // (rounded) x * g of channel_conv1's gate pass, else t gated in the
    // epilogue.
    if (has_se && gated.buf >= 0) {
      e2.res = &gated;
    } else {
      e2.res = &t;
      if (has_se) e2.res_gate = &gate;
    }
  }
  return B.conv(h, c2, e2, p + ".channel_conv2");
}

// LargeStem (src/cpu/model.rs:626-693): the max-pool and stem2b write the two
// halves of the concat stem3 reads.
View large_stem(Builder& B, const View& x, int mid, int out) {
  std::string p = "model.backbone.encoder.convolution";
  Epi relu;
  relu.act = ACT_RELU;
  ConvW s1 = B.conv_w(p + ".stem1", 3, mid, 3, 3, 2, 2, {1, 1, 1, 1}, false, "normalization", 4);
  View e = B.conv(x, s1, relu, p + ".stem1");
  ConvW s2a = B.conv_w(p + ".stem2a", mid, mid / 2, 2, 2, 1, 1, {0, 0, 1, 1}, false, "normalization");
  View a = B.conv(e, s2a, relu, p + ".stem2a");
  View merged = B.alloc(e.n, e.h, e.w, 2 * mid, p + ".concat");
  View pooled_slot = Builder::slice(merged, 0, mid);
  View branch_slot = Builder::slice(merged, mid, mid);
  B.maxpool_same(e, pooled_slot, p + ".pool");
  ConvW s2b = B.conv_w(p + ".stem2b", mid / 2, mid, 2, 2, 1, 1, {0, 0, 1, 1}, false, "normalization");
  Epi into = relu;
  into.dst = &branch_slot;
  B.conv(a, s2b, into, p + ".stem2b");
  ConvW s3 = B.conv_w(p + ".stem3", 2 * mid, mid, 3, 3, 2, 2, {1, 1, 1, 1}, false, "normalization");
  View t = B.conv(merged, s3, relu, p + ".stem3");
  ConvW s4 = B.conv_w(p + ".stem4", mid, out, 1, 1, 1, 1, {0, 0, 0, 0}, false, "normalization");
  return B.conv(t, s4, relu, p + ".stem4");
}

// SmallStem (src/cpu/model.rs:695-733): 3x3 s2 BN GELU, 3x3 s2 BN.
View small_stem(Builder& B, const View& x, int mid, int out) {
  std::string p = "model.backbone.encoder.convolution";
  ConvW c1 = B.conv_w(p + ".conv1", 3, mid, 3, 3, 2, 2, {1, 1, 1, 1}, false, "normalization", 4);
  Epi gelu;
  gelu.act = ACT_GELU;
  View h = B.conv(x, c1, gelu, p + ".conv1");
  ConvW c2 = B.conv_w(p + ".conv2", mid, out, 3, 3, 2, 2, {1, 1, 1, 1}, false, "normalization");
  return B.conv(h, c2, Epi{}, p + ".conv2");
}

std::vector<View> backbone(Builder& B, const View& x, int mid, int out, bool large,
                           const std::vector<std::vector<BlockSpec>>& stages) {
  View h = large ? large_stem(B, x, mid, out) : small_stem(B, x, mid, out);
  std::vector<View> outs;
  for (size_t s = 0; s < stages.size(); ++s) {
    for (size_t b = 0; b < stages[s].size(); ++b)
      h = lcnet_block(B, h, "model.backbone.encoder.blocks." + std::to_string(s) + ".blocks." + std::to_string(b),
                      stages[s][b]);
    outs.push_back(h);
  }
  return outs;
}

// detector_stages_for_channels (src/cpu/model.rs:1648-1673).
std::vector<std::vector<BlockSpec>> detector_stages(const int c[4]) {
  return {{{c[0], c[0], 1, 1, true}, {c[0], c[0], 1, 1, false}},
          {{c[0], c[1], 2, 2, false}, {c[1], c[1], 1, 1, true}, {c[1], c[1], 1, 1, false}},
          {{c[1], c[2], 2, 2, false},
           {c[2], c[2], 1, 1, true},
           {c[2], c[2], 1, 1, false},
           {c[2], c[2], 1, 1, true},
           {c[2], c[2], 1, 1, false}},
          {{c[2], c[3], 2, 2, false}, {c[3], c[3], 1, 1, true}, {c[3], c[3], 1, 1, false}}};
}

// recognizer stage tables (src/cpu/model.rs:2057-2122).
std::vector<std::vector<BlockSpec>> recognizer_stages(int size) {
  auto alt = [](std::vector<BlockSpec> v, int c) {
    for (int i = 0; i < 6; ++i) v.push_back({c, c, 1, 1, i % 2 == 0});
    return v;
  };
  if (size == PPOCR_SIZE_MEDIUM)
    return {{{128, 128, 1, 1, true}},
            {{128, 256, 1, 1, false}, {256, 256, 1, 1, false}, {256, 256, 1, 1, true}},
            alt({{256, 512, 2, 1, false}}, 512),
            {{512, 768, 2, 1, false}, {768, 768, 1, 1, true}, {768, 768, 1, 1, false}}};
  if (size == PPOCR_SIZE_SMALL)
    return {{{96, 96, 1, 1, true}},
            {{96, 96, 1, 1, false}, {96, 96, 1, 1, false}},
            alt({{96, 192, 2, 1, false}}, 192),
            {{192, 384, 2, 1, false}, {384, 384, 1, 1, true}, {384, 384, 1, 1, false}}};
  return {{{48, 48, 1, 1, true}},
          {{48, 48, 1, 1, false}},
          {{48, 96, 2, 1, false}, {96, 96, 1, 1, true}, {96, 96, 1, 1, false}},
          {{96, 160, 2, 1, false}, {160, 160, 1, 1, true}, {160, 160, 1, 1, false}, {160, 160, 1, 1, false}}};
}

// ------------------------------------------------------------------ necks

// RepLkFpn (src/cpu/model.rs:1197-1254).  Level i of the concat goes to
// channel slot 3 - i (deepest first) upsampled by 2^i.
View rep_lk_fpn(Builder& B, const std::vector<View>& st, const int chans[4], int nc, int k) {
  const int q = nc / 4;
  std::vector<View> h(4), fused(4);
  std::vector<Builder::SePartial> sums(4);
  std::vector<SeW> sws(4);
  // The four levels' insert convs in one launch where they share a kernel.
  std::vector<const View*> ins(4);
  std::vector<ConvW> iw(4);
  std::vector<std::string> inames(4);
  for (int i = 0; i < 4; ++i) {
    std::string p = "model.neck.insert_conv." + std::to_string(i);
    ins[i] = &st[i];
    iw[i] = B.conv_w(p + ".in_conv", chans[i], nc, 1, 1, 1, 1, {0, 0, 0, 0}, false);
    inames[i] = p + ".in_conv";
    sws[i] = B.se_w(p + ".squeeze_excitation_block.conv1", p + ".squeeze_excitation_block.conv2", nc, nc / 4,
                    ACT_HSIG5);
  }
  h = B.conv_levels(ins, iw, Epi{}, inames, "model.neck.insert_conv.in_conv", &sums);
  // The four levels' gates (each from its conv's channel sums) in one launch.
  std::vector<View> g = B.se_levels(h, sws, "model.neck.insert_conv.se", sums);
  // fused[i] = h + h * g (+ up2(fused[i + 1])) feeds input_conv i's
  // depthwise and level i - 1.  Where the depthwise can form it from h in its
  // tile loads, levels run deepest first and the depthwise also stores it for
  // the next level (level 0's is read by nothing else and is not stored);
  // otherwise gate_residual writes every level first.
  int pd = k / 2;
  bool gr_fused = true;
  for (int i = 0; i < 4; ++i)
    gr_fused = gr_fused && depthwise_gate_residual_supported(k, k, 1, 1) &&
               (i == 3 || (h[i].h == 2 * h[i + 1].h && h[i].w == 2 * h[i + 1].w));
  if (!gr_fused)
    for (int i = 3; i >= 0; --i) {
      fused[i] = B.alloc(h[i].n, h[i].h, h[i].w, nc, "model.neck.fused." + std::to_string(i));
      B.gate_residual(h[i], g[i], i < 3 ? &fused[i + 1] : nullptr, fused[i], 1,
                      "model.neck.fused." + std::to_string(i));
    }
  View cat = B.alloc(h[0].n, h[0].h, h[0].w, nc, "model.neck.concat");
  std::vector<DwW> dws(4);
  for (int i = 0; i < 4; ++i)
    dws[i] = B.dw_w("model.neck.input_conv." + std::to_string(i) + ".depthwise_convolution", nc, k, k, 1, 1,
                    {pd, pd, pd, pd}, true);
  std::vector<View> d(4);
  if (gr_fused)
    for (int i = 3; i >= 0; --i) {
      if (i > 0) fused[i] = B.alloc(h[i].n, h[i].h, h[i].w, nc, "model.neck.fused." + std::to_string(i));
      Builder::GateResidual gr;
      gr.gate = g[i];
      gr.upper = i < 3 ? &fused[i + 1] : nullptr;
      gr.out = i > 0 ? &fused[i] : nullptr;
      gr.name = "model.neck.fused." + std::to_string(i);
      d[i] = B.depthwise(h[i], dws[i], ACT_NONE, nullptr, "model.neck.input_conv." + std::to_string(i) +
                         ".depthwise_convolution", 0, nullptr, &gr);
    }
  std::vector<View> pt(4), slots(4);
  std::vector<Builder::SePartial> psums(4);
  std::vector<SeW> psw(4);
  std::vector<int> reps(4);
  std::vector<const View*> pin(4);
  std::vector<ConvW> pws(4);
  std::vector<std::string> pnames(4);
  for (int i = 0; i < 4; ++i) {
    std::string p = "model.neck.input_conv." + std::to_string(i);
    if (!gr_fused) d[i] = B.depthwise(fused[i], dws[i], ACT_NONE, nullptr, p + ".depthwise_convolution");
    pin[i] = &d[i];
    pws[i] = B.conv_w(p + ".pointwise_convolution", nc, q, 1, 1, 1, 1, {0, 0, 0, 0}, false);
    pnames[i] = p + ".pointwise_convolution";
    psw[i] = B.se_w(p + ".squeeze_excitation_module.conv1", p + ".squeeze_excitation_module.conv2", q, q / 4,
                    ACT_HSIG5);
    slots[i] = Builder::slice(cat, (3 - i) * q, q);
    reps[i] = 1 << i;
  }
  // The four pointwise convs in one launch where they share a kernel.
  pt = B.conv_levels(pin, pws, Epi{}, pnames, "model.neck.input_conv.pointwise_convolution", &psums);
  // Every level's gate, then every level's x + x*g written upsampled into
  // its concat slot (deepest first in the channels): one launch each.
  std::vector<View> gi = B.se_levels(pt, psw, "model.neck.input_conv.se", psums);
  std::vector<std::string> level_names;
  for (int i = 0; i < 4; ++i) level_names.push_back("model.neck.input_conv." + std::to_string(i) + ".out");
  B.gate_residual_levels(pt, gi, slots, reps, "model.neck.input_conv.out", level_names);
  return cat;
}

// factor_rank_one_conv_weight (src/cpu/model.rs:221-369): per input channel,
// four power iterations in double precision on the O x k^2 matrix, then the
// separability check.  Returns dw [ci][k*k] and pw [co][ci].
void factor_rank_one(const std::string& name, const std::vector<float>& W, int ci, int co, int k,
                     std::vector<float>& dw, std::vector<float>& pw) {
  const int sp = k * k;
  for (float v : W)
    if (!std::isfinite(v)) raise(PPOCR_ERR_INVALID_MODEL, name + ": rank-one weight contains non-finite values");
  dw.assign((size_t)ci * sp, 0.0f);
  pw.assign((size_t)co * ci, 0.0f);
  std::vector<double> dir(sp), sc(co);
  auto at = [&](int o, int c, int i) { return (double)W[((size_t)o * ci + c) * sp + i]; };
  for (int c = 0; c < ci; ++c) {
    int best = 0;
    double best_e = 0.0;
    for (int o = 0; o < co; ++o) {
      double e = 0.0;
      for (int i = 0; i < sp; ++i) e += at(o, c, i) * at(o, c, i);
      if (e > best_e) best = o, best_e = e;
    }
    if (best_e == 0.0) continue;
    double nrm = std::sqrt(best_e);
    for (int i = 0; i < sp; ++i) dir[i] = at(best, c, i) / nrm;
    for (int it = 0; it < 4; ++it) {
      double energy = 0.0;
      for (int o = 0; o < co; ++o) {
        double s = 0.0;
        for (int i = 0; i < sp; ++i) s += at(o, c, i) * dir[i];
        sc[o] = s;
        energy += s * s;
      }
      if (!(std::isfinite(energy) && energy > 0.0))
        raise(PPOCR_ERR_INVALID_MODEL, name + ": rank-one factorization became degenerate");
      double n2 = 0.0;
      for (int i = 0; i < sp; ++i) {
        double s = 0.0;
        for (int o = 0; o < co; ++o) s += at(o, c, i) * sc[o];
        dir[i] = s / energy;
        n2 += dir[i] * dir[i];
      }
      n2 = std::sqrt(n2);
      if (!(std::isfinite(n2) && n2 > 0.0))
        raise(PPOCR_ERR_INVALID_MODEL, name + ": rank-one spatial factor became degenerate");
      for (int i = 0; i < sp; ++i) dir[i] /= n2;
    }
    for (int o = 0; o < co; ++o) {
      double s = 0.0;
      for (int i = 0; i < sp; ++i) s += at(o, c, i) * dir[i];
      pw[(size_t)o * ci + c] = (float)s;
    }
    for (int i = 0; i < sp; ++i) dw[(size_t)c * sp + i] = (float)dir[i];
  }
  double max_src = 0, max_err = 0, src_e = 0, err_e = 0;
  for (int o = 0; o < co; ++o)
    for (int c = 0; c < ci; ++c)
      for (int i = 0; i < sp; ++i) {
        float e = W[((size_t)o * ci + c) * sp + i];
        float a = pw[(size_t)o * ci + c] * dw[(size_t)c * sp + i];
        double err = std::fabs((double)(e - a));
        max_src = std::max(max_src, (double)std::fabs(e));
        max_err = std::max(max_err, err);
        src_e += (double)e * e;
        err_e += err * err;
      }
  double rel = src_e == 0.0 ? 0.0 : std::sqrt(err_e / src_e);
  if (!(max_err <= max_src * 1e-5 + 1e-12 && rel <= 1e-6))
    raise(PPOCR_ERR_INVALID_MODEL, name + ": fused convolution is not rank-one separable");
}

// RankOneConv2d (src/cpu/model.rs:165-219): depthwise k x k then 1x1 + bias.
struct RankOneW {
  DwW dw;
  ConvW pw;
};

RankOneW rank_one_w(Builder& B, const std::string& p, int ci, int co, int k) {
  std::vector<float> W = B.get(p + ".weight", {co, ci, k, k}).v;
  std::vector<float> dwv, pwv;
  factor_rank_one(p, W, ci, co, k, dwv, pwv);
  int pd = k / 2;
  RankOneW r;
  r.dw = B.pack_dw(dwv, {}, ci, k, k, 1, 1, {pd, pd, pd, pd});
  r.pw = B.pack_conv(pwv, B.get(p + ".bias", {co}).v, ci, co, 1, 1, 1, 1, {0, 0, 0, 0});
  return r;
}

// The rank-one convs of the four neck levels: the depthwise layers one by
// one, the pointwise layers as one launch where they can share one.
std::vector<View> rank_one_levels(Builder& B, const std::vector<View>& xs, const std::string& prefix, int ci, int co,
                                  int k) {
  std::vector<View> d(4);
  std::vector<const View*> dp(4);
  std::vector<ConvW> pws(4);
  std::vector<std::string> names(4);
  for (int i = 0; i < 4; ++i) {
    const std::string p = prefix + "." + std::to_string(i);
    const RankOneW r = rank_one_w(B, p, ci, co, k);
    d[i] = B.depthwise(xs[i], r.dw, ACT_NONE, nullptr, p + ".depthwise");
    dp[i] = &d[i];
    pws[i] = r.pw;
    names[i] = p + ".pointwise";
  }
  return B.conv_levels(dp, pws, Epi{}, names, prefix + ".pointwise");
}

// fuse_intraclass_conv (src/cpu/model.rs:819-906).
ConvW intraclass_conv(Builder& B, const std::string& p, const std::string& ratio, int k) {
  std::vector<float> W = B.get(p + ".symmetric_conv_long_" + ratio + ".weight", {32, 32, k, k}).v;
  std::vector<float> b = B.get(p + ".symmetric_conv_long_" + ratio + ".bias", {32}).v;
  std::vector<float> vw = B.get(p + ".vertical_long_to_small_conv_" + ratio + ".weight", {32, 32, k, 1}).v;
  std::vector<float> vb = B.get(p + ".vertical_long_to_small_conv_" + ratio + ".bias", {32}).v;
  std::vector<float> hw = B.get(p + ".horizontal_small_to_long_conv_" + ratio + ".weight", {32, 32, 1, k}).v;
  std::vector<float> hb = B.get(p + ".horizontal_small_to_long_conv_" + ratio + ".bias", {32}).v;
  int ctr = k / 2;
  for (int o = 0; o < 32; ++o)
    for (int i = 0; i < 32; ++i) {
      size_t bo = ((size_t)o * 32 + i) * k;
      for (int r = 0; r < k; ++r) W[bo * k + r * k + ctr] += vw[bo + r];
      for (int c = 0; c < k; ++c) W[bo * k + ctr * k + c] += hw[bo + c];
    }
  for (int o = 0; o < 32; ++o) {
    b[o] += vb[o];
    b[o] += hb[o];
  }
  return B.pack_conv(W, b, 32, 32, k, k, 1, 1, {ctr, ctr, ctr, ctr});
}

// DetectorNeck, medium (src/cpu/model.rs:948-1067).
View medium_neck(Builder& B, const std::vector<View>& st) {
  const int chans[4] = {128, 256, 512, 896};
  std::string n = "model.neck";
  std::vector<View> td(4);
  for (int i = 3; i >= 0; --i) {
    std::string p = n + ".input_channel_adjustment_convolution." + std::to_string(i);
    ConvW w = B.conv_w(p, chans[i], 256, 1, 1, 1, 1, {0, 0, 0, 0}, false);
    Epi e;
    if (i < 3) e.up = &td[i + 1];
    td[i] = B.conv(st[i], w, e, p);
  }
  // The projections of the four levels, then the bottom-up chain
  // p[i] += conv3x3s2(p[i - 1]) (the projection added in the pan conv's
  // epilogue).
  std::vector<View> proj = rank_one_levels(B, td, n + ".input_feature_projection_convolution", 256, 64, 9);
  std::vector<View> bu(4);
  for (int i = 0; i < 4; ++i) {
    if (i == 0) {
      bu[i] = proj[0];
    } else {
      std::string p = n + ".path_aggregation_head_convolution." + std::to_string(i - 1);
      ConvW w = B.conv_w(p, 64, 64, 3, 3, 2, 2, {1, 1, 1, 1}, false);
      Epi e;
      e.res = &proj[i];
      bu[i] = B.conv(bu[i - 1], w, e, p);
    }
  }
  const View& b0 = bu[0];
  View cat = B.alloc(b0.n, b0.h, b0.w, 256, n + ".concat");
  std::vector<View> lat = rank_one_levels(B, bu, n + ".path_aggregation_lateral_convolution", 64, 64, 9);
  // IntraclassBlock per level, each step of the four levels as one launch
  // where they can share one: 1x1 64 -> 32, the fused 7x7, 5x5 and 3x3, then
  // conv_final (upsampled into the concat slot, one launch per level).
  auto step = [&](const std::vector<View>& xs, auto make_w, const std::string& suffix) {
    std::vector<const View*> xp(4);
    std::vector<ConvW> ws(4);
    std::vector<std::string> names(4);
    for (int i = 0; i < 4; ++i) {
      const std::string p = n + ".intraclass_blocks." + std::to_string(i);
      xp[i] = &xs[i];
      ws[i] = make_w(p);
      names[i] = p + suffix;
    }
    return B.conv_levels(xp, ws, Epi{}, names, n + ".intraclass_blocks" + suffix);
  };
  std::vector<View> r = step(lat, [&](const std::string& p) {
    return B.conv_w(p + ".conv_reduce_channel", 64, 32, 1, 1, 1, 1, {0, 0, 0, 0}, true);
  }, ".conv_reduce_channel");
  std::vector<View> l7 = step(r, [&](const std::string& p) { return intraclass_conv(B, p, "longratio", 7); }, ".long");
  std::vector<View> l5 = step(l7, [&](const std::string& p) { return intraclass_conv(B, p, "midratio", 5); }, ".mid");
  std::vector<View> l3 = step(l5, [&](const std::string& p) { return intraclass_conv(B, p, "shortratio", 3); }, ".short");
  for (int i = 0; i < 4; ++i) {
    std::string p = n + ".intraclass_blocks." + std::to_string(i);
    ConvW fin = B.conv_w(p + ".conv_final", 32, 64, 1, 1, 1, 1, {0, 0, 0, 0}, true, "norm");
    View slot = Builder::slice(cat, (3 - i) * 64, 64);
    Epi e;
    e.act = ACT_RELU;
    e.res = &lat[i];
    e.rep = 1 << i;
    e.dst = &slot;
    B.conv(l3[i], fin, e, p + ".conv_final");
  }
  return cat;
}

// DetectorHead (src/cpu/model.rs:1479-1521).
void detector_head(Builder& B, const View& x, int nc) {
  int h = nc / 4;
  if (h != 16 && h != 24 && h != 64) raise(PPOCR_ERR_INVALID_MODEL, "unsupported detector head width");
  ConvW down = B.conv_w("head.conv_down", nc, h, 3, 3, 1, 1, {1, 1, 1, 1}, false, "norm");
  Epi relu;
  relu.act = ACT_RELU;
  View d = B.conv(x, down, relu, "head.conv_down");
  std::vector<float> wu = B.get("head.conv_up.convolution.weight", {h, h, 2, 2}).v;
  std::vector<float> bu = B.get("head.conv_up.convolution.bias", {h}).v;
  B.fold_bn(wu, bu, "head.conv_up.norm", h, true, h);
  // conv_up's weights are bf16 in a bf16 plan on both of its kernels (the
  // matrix-core GEMM takes them so; the vector-ALU kernel reads the same
  // bf16 values in fp32).
  if (B.dt() == DT_BF16)
    for (float& v : wu) v = bf16_value(v);
  std::vector<float> wf = B.get("head.conv_final.weight", {h, 1, 2, 2}).v;
  float bf = B.get("head.conv_final.bias", {1}).v[0];
  size_t owu = B.put(wu), obu = B.put(bu), owf = B.put(wf);
  Plan& plan = B.plan();
  View out = B.alloc(x.n, 4 * d.h, 4 * d.w, 1, "output", DT_F32);
  plan.output = out.buf;
  plan.output_elems = out.pixels();
  plan.output_shape = {(size_t)x.n, 1, (size_t)out.h, (size_t)out.w};
  View in = d;
  Op op;
  op.name = "head.conv_up+conv_final";
  if (B.dt() == DT_BF16) op.bf16_weights = {"head.conv_up"};
  op.flops = 2.0 * d.pixels() * (4.0 * h * h + 16.0 * h);
  op.bytes = (double)dtype_size(d.dt) * d.pixels() * h + 4.0 * ((double)out.pixels() + 4.0 * h * h + 4.0 * h);
  op.reads = {d.buf};
  op.writes = {out.buf};
  const int M = d.n * d.h * d.w;
  if (conv_tile_cols(M, 4 * h, d.dt) % h == 0) {
    // conv_up on the matrix cores as a 1x1 conv with 4h columns (column
    // tap * h + o, weight wu[c][o][tap], bias bu[o]); conv_final and the
    // sigmoid run in its epilogue (tiles are whole taps wide).
    std::vector<float> w1((size_t)4 * h * h), b1((size_t)4 * h);
    for (int tap = 0; tap < 4; ++tap)
      for (int o = 0; o < h; ++o) {
        b1[(size_t)tap * h + o] = bu[o];
        for (int c = 0; c < h; ++c) w1[((size_t)tap * h + o) * h + c] = wu[((size_t)c * h + o) * 4 + tap];
      }
    const ConvW up = B.pack_conv(w1, b1, h, 4 * h, 1, 1, 1, 1, {0, 0, 0, 0});
    ConvParams base{};
    base.N = d.n, base.H = d.h, base.W = d.w, base.C = d.c, base.in_ps = d.ps;
    base.Ho = d.h, base.Wo = d.w, base.Co = 4 * h, base.out_ps = 1;
    base.out_f32 = 1;
    base.ldw = up.ldw;
    base.kh = base.kw = base.sh = base.sw = 1;
    base.act = ACT_RELU;
    base.up_s = 2;
    base.rep = 1;
    base.out_h = out.h, base.out_w = out.w;
    base.dt = d.dt;
    base.db_ch = h;
    base.db_bf = bf;
    const size_t uw = up.w, ub = up.b;
    op.kernel = Builder::conv_kernel(base, d, uw, false) + "+db_head";
    op.bound = 1;
    op.launch = [=](const Exec& ex, hipStream_t s) {
      ConvParams p = base;
      p.in = ex.ptr(in);
      p.out = ex.fptr(out);
      p.wt = ex.wv(uw);
      p.bias = ex.w(ub);
      p.db_wf = ex.w(owf);
      launch_conv(p, s);
    };
  } else {
    op.kernel = "db_head_up";
    op.launch = [=](const Exec& ex, hipStream_t s) {
      launch_db_head_up(ex.ptr(in), in.n, in.h, in.w, in.c, in.ps, ex.w(owu), ex.w(obu), ex.w(owf), bf, ex.fptr(out),
                        in.dt, s);
    };
  }
  B.add_op(std::move(op));
}

void validate_detector_shape(const size_t s[4]) {
  if (s[0] == 0 || s[1] != 3 || s[2] < 32 || s[3] < 32 || s[2] % 32 || s[3] % 32)
    raise(PPOCR_ERR_INVALID_INPUT,
          "detector expects [N, 3, H, W] with N > 0, H/W >= 32 and divisible by 32; got [" + std::to_string(s[0]) +
              ", " + std::to_string(s[1]) + ", " + std::to_string(s[2]) + ", " + std::to_string(s[3]) + "]");
  // Larger batches run in chunks sized to the per-buffer limit; one image's
  // buffers must fit it on their own.
  if (s[0] > (1u << 24) || s[2] > (1u << 15) || s[3] > (1u << 15))
    raise(PPOCR_ERR_INVALID_INPUT, "detector input shape is too large");
}

void validate_recognizer_shape(const size_t s[4]) {
  if (s[0] == 0 || s[1] != 3 || s[2] != 48 || s[3] < 32 || s[3] % 4)
    raise(PPOCR_ERR_INVALID_INPUT,
          "recognizer expects [N, 3, 48, W] with N > 0, W >= 32 and divisible by 4; got [" + std::to_string(s[0]) +
              ", " + std::to_string(s[1]) + ", " + std::to_string(s[2]) + ", " + std::to_string(s[3]) + "]");
  // The reference bounds a rectified crop to a 4096-px edge (src/ocr.rs:20,
  // :1145-1156), i.e. canvases up to 48 * 4096 = 196608 px; one line's
  // buffers fit the per-buffer limit up to about 229000 px, larger batches
  // run in chunks.
  if (s[0] > (1u << 24) || s[3] > (1u << 18))
    raise(PPOCR_ERR_INVALID_INPUT, "recognizer input shape is too large");
}

}  // namespace

// Detector::load (src/gpu/model.rs:50-93; architecture src/cpu/model.rs:1546-1609).
Plan build_detector(const SafeTensors& st, int size, const size_t nchw[4], int dt) {
  validate_detector_shape(nchw);
  const size_t expected = size == PPOCR_SIZE_MEDIUM ? 350 : 271;
  const char* tier = size == PPOCR_SIZE_MEDIUM ? "medium" : size == PPOCR_SIZE_SMALL ? "small" : "tiny";
  if (st.size() != expected)
    raise(PPOCR_ERR_INVALID_MODEL, std::string(tier) + " detector has " + std::to_string(st.size()) +
                                       " tensors; expected " + std::to_string(expected));
  Plan plan;
  plan.detector = true;
  Builder B(st, plan, dt);
  int chans[4], mid, out, nc;
  if (size == PPOCR_SIZE_MEDIUM) {
    const int c[4] = {128, 256, 512, 896};
    std::copy(c, c + 4, chans);
    mid = 64, out = 128, nc = 256;
  } else if (size == PPOCR_SIZE_SMALL) {
    const int c[4] = {48, 96, 192, 384};
    std::copy(c, c + 4, chans);
    mid = 24, out = 48, nc = 96;
  } else {
    const int c[4] = {32, 48, 64, 160};
    std::copy(c, c + 4, chans);
    mid = 16, out = 32, nc = 64;
  }
  View x = B.input(nchw);
  std::vector<View> stages = backbone(B, x, mid, out, true, detector_stages(chans));
  View neck = size == PPOCR_SIZE_MEDIUM ? medium_neck(B, stages)
                                        : rep_lk_fpn(B, stages, chans, nc, size == PPOCR_SIZE_SMALL ? 7 : 5);
  detector_head(B, neck, nc);
  plan_arena(plan);
  return plan;
}

// Recognizer::load (src/gpu/model.rs:156-220; architecture
// src/cpu/model.rs:1961-2039).
Plan build_recognizer(const SafeTensors& st, int size, const size_t nchw[4], int dt, bool greedy) {
  validate_recognizer_shape(nchw);
  const size_t expected = size == PPOCR_SIZE_MEDIUM ? 269 : size == PPOCR_SIZE_SMALL ? 250 : 150;
  const char* tier = size == PPOCR_SIZE_MEDIUM ? "medium" : size == PPOCR_SIZE_SMALL ? "small" : "tiny";
  if (st.size() != expected)
    raise(PPOCR_ERR_INVALID_MODEL, std::string(tier) + " recognizer has " + std::to_string(st.size()) +
                                       " tensors; expected " + std::to_string(expected));
  Plan plan;
  plan.detector = false;
  Builder B(st, plan, dt);
  View x = B.input(nchw);
  bool tiny = size == PPOCR_SIZE_TINY;
  int mid = size == PPOCR_SIZE_MEDIUM ? 64 : size == PPOCR_SIZE_SMALL ? 48 : 24;
  int out = size == PPOCR_SIZE_MEDIUM ? 128 : size == PPOCR_SIZE_SMALL ? 96 : 48;
  std::vector<View> stages = backbone(B, x, mid, out, !tiny, recognizer_stages(size));
  View pooled = B.avgpool32(stages.back(), "pool");
  if (pooled.h != 1) raise(PPOCR_ERR_INVALID_MODEL, "recognizer pooling must produce height 1");
  const int classes = tiny ? 6906 : 18710;
  View feat;  // classifier input [N, 1, T, C]
  ConvW cls;
  std::string cls_name;
  if (tiny) {
    // TinyRecognizerHead (src/cpu/model.rs:1913-1936) with Conv1dBn (:1877-1911).
    std::vector<float> w1 = B.get("head.conv1.weight", {160, 1, 5}).v, b1;
    B.fold_bn(w1, b1, "head.norm1", 160);
    DwW dw = B.pack_dw(w1, b1, 160, 1, 5, 1, 1, {0, 2, 0, 2});
    View h = B.depthwise(pooled, dw, ACT_HSWISH, nullptr, "head.conv1");
    std::vector<float> w2 = B.get("head.conv2.weight", {160, 160, 1}).v, b2;
    B.fold_bn(w2, b2, "head.norm2", 160);
    ConvW c2 = B.pack_conv(w2, b2, 160, 160, 1, 1, 1, 1, {0, 0, 0, 0});
    Epi hs;
    hs.act = ACT_HSWISH;
    h = B.conv(h, c2, hs, "head.conv2");
    feat = B.conv(h, B.linear_w("head.fc1", 160, 80), Epi{}, "head.fc1");
    cls = B.linear_w("head.fc2", 80, classes);
    cls_name = "head.fc2";
  } else {
    // LightSvtrRecognizerHead / RecEncoder (src/cpu/model.rs:1686-1875).
    int ci = size == PPOCR_SIZE_MEDIUM ? 768 : 384;
    int hid = size == PPOCR_SIZE_MEDIUM ? 192 : 120;
    int mlp = size == PPOCR_SIZE_MEDIUM ? 768 : 240;
    std::string e = "head.encoder";
    Epi silu;
    silu.act = ACT_SILU;
    View skip = B.conv(pooled, B.conv_w(e + ".conv_block.0", ci, hid, 1, 1, 1, 1, {0, 0, 0, 0}, false, "normalization"),
                       silu, e + ".conv_block.0");
    View h = B.conv(pooled, B.conv_w(e + ".conv_block.1", ci, hid, 1, 1, 1, 1, {0, 0, 0, 0}, false, "normalization"),
                    silu, e + ".conv_block.1");
    DwW lw = B.dw_w(e + ".conv_block.2", hid, 1, 7, 1, 1, {0, 3, 0, 3}, false, "normalization");
    h = B.depthwise(h, lw, ACT_SILU, &h, e + ".conv_block.2");
    for (int i = 0; i < 2; ++i) {
      std::string p = e + ".svtr_block." + std::to_string(i);
      // fp32 plans fuse each block LayerNorm into the linear layer after it.
      const bool fuse_ln = ln_linear_supported(hid, 3 * hid, B.dt()) && ln_linear_supported(hid, mlp, B.dt());
      ConvW qkv_w = B.linear_w(p + ".self_attn.qkv", hid, 3 * hid);
      View qkv = fuse_ln ? B.ln_linear(h, p + ".layer_norm1", qkv_w, ACT_NONE, p + ".layer_norm1+qkv")
                         : B.conv(B.layer_norm(h, p + ".layer_norm1", nullptr, p + ".layer_norm1"), qkv_w, Epi{},
                                  p + ".self_attn.qkv");
      View ctx = B.attention(qkv, hid, 8, p + ".self_attn");
      Epi r1;
      r1.res = &h;
      View h1 = B.conv(ctx, B.linear_w(p + ".self_attn.projection", hid, hid), r1, p + ".self_attn.projection");
      ConvW fc1_w = B.linear_w(p + ".mlp.fc1", hid, mlp);
      View m = fuse_ln ? B.ln_linear(h1, p + ".layer_norm2", fc1_w, ACT_SILU, p + ".layer_norm2+fc1")
                       : B.conv(B.layer_norm(h1, p + ".layer_norm2", nullptr, p + ".layer_norm2"), fc1_w, silu,
                                p + ".mlp.fc1");
      Epi r2;
      r2.res = &h1;
      h = B.conv(m, B.linear_w(p + ".mlp.fc2", mlp, hid), r2, p + ".mlp.fc2");
    }
    feat = B.layer_norm(h, e + ".norm", &skip, e + ".norm");
    cls = B.linear_w("head.head", hid, classes);
    cls_name = "head.head";
  }
  const size_t n = (size_t)pooled.n, steps = (size_t)pooled.w;
  if (greedy) {
    View out = B.greedy_classifier(feat, cls, cls_name);
    plan.output = out.buf;
    plan.output_elems = n * steps * 2;
    plan.output_shape = {n, steps, 2};
  } else {
    View logits = B.alloc(pooled.n, 1, pooled.w, classes, "output", DT_F32);
    plan.output = logits.buf;
    plan.output_elems = n * steps * classes;
    plan.output_shape = {n, steps, (size_t)classes};
    Epi into;
    into.dst = &logits;
    B.conv(feat, cls, into, cls_name);
    B.softmax(logits, "softmax");
  }
  plan_arena(plan);
  return plan;
}

// Interval packing of buffer lifetimes: largest first, each at the lowest
// offset that overlaps no placed buffer whose lifetime intersects its own.
void plan_arena(Plan& plan) {
  const int end = (int)plan.ops.size();
  for (auto& b : plan.bufs) {
    if (b.first < 0) b.first = b.last = 0;
  }
  plan.bufs[plan.staging].first = 0;
  plan.bufs[plan.output].last = end;
  std::vector<int> order(plan.bufs.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = (int)i;
  std::sort(order.begin(), order.end(), [&](int a, int b) {
    if (plan.bufs[a].bytes != plan.bufs[b].bytes) return plan.bufs[a].bytes > plan.bufs[b].bytes;
    return a < b;
  });
  std::vector<int> placed;
  size_t total = 0, unplanned = 0;
  for (int id : order) {
    Buffer& b = plan.bufs[id];
    size_t size = round_up(b.bytes, 256);
    unplanned += size;
    std::vector<std::pair<size_t, size_t>> busy;
    for (int o : placed) {
      const Buffer& q = plan.bufs[o];
      if (q.first <= b.last && b.first <= q.last) busy.push_back({q.arena_off, q.arena_off + round_up(q.bytes, 256)});
    }
    std::sort(busy.begin(), busy.end());
    size_t off = 0;
    for (auto& r : busy) {
      if (r.first >= off + size) break;
      off = std::max(off, r.second);
    }
    b.arena_off = off;
    total = std::max(total, off + size);
    placed.push_back(id);
  }
  plan.arena_bytes = total;
  plan.unplanned_bytes = unplanned;
}

std::vector<std::string> plan_rounding_points(const Plan& plan) {
  std::vector<std::string> out;
  if (plan.dt != DT_BF16) return out;
  std::vector<int> writers(plan.bufs.size(), 0);
  for (const Op& op : plan.ops)
    for (int b : op.writes) ++writers[b];
  for (const Op& op : plan.ops) {
    if (op.rounds_set) {
      for (const std::string& r : op.rounds) out.push_back("A " + r);
    } else if (!op.exact) {
      for (int b : op.writes)
        if (plan.bufs[b].dt == DT_BF16) out.push_back("A " + (writers[b] == 1 ? plan.bufs[b].name : op.name));
    }
    for (const std::string& w : op.bf16_weights) out.push_back("W " + w);
  }
  return out;
}

}  // namespace ppocr
