// Test harness for the convolution kernels, built as libppocr_hip_probe.so
// next to the backend and loaded only by tests/: one launch_conv on host
// arrays, with the split count, storage type and SE input gate chosen by the
// caller, so every kernel variant (1x1 / k x k, direct / register-staged,
// gated, split K, bf16) can be checked against a CPU convolution on shapes
// that exercise its tails.  Not part of the backend's C ABI.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <vector>

#include "kernels.h"
#include "runtime.h"

namespace {

uint16_t to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);  // NaN stays NaN
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

float from_bf16(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// Device copy of n floats, stored as fp32 or (dt = bf16) rounded to bf16.
void* upload(const float* src, size_t n, int dt) {
  void* d = nullptr;
  if (dt == ppocr::DT_BF16) {
    std::vector<uint16_t> h(n);
    for (size_t i = 0; i < n; ++i) h[i] = to_bf16(src[i]);
    if (hipMalloc(&d, n * 2) != hipSuccess) return nullptr;
    if (hipMemcpy(d, h.data(), n * 2, hipMemcpyHostToDevice) != hipSuccess) return nullptr;
  } else {
    if (hipMalloc(&d, n * 4) != hipSuccess) return nullptr;
    if (hipMemcpy(d, src, n * 4, hipMemcpyHostToDevice) != hipSuccess) return nullptr;
  }
  return d;
}

// ppocr_probe_conv, and with se_rows the SE channel sums the conv leaves:
// *se_rows = conv_se_blocks() and se_part [*se_rows][co] (when non-zero).
int run_conv(const float* x, int n, int h, int w, int c, const float* weight, const float* bias, int co, int kh,
             int kw, int sh, int sw, int pt, int pl, int pb, int pr, int act, const float* gate, int splits, int dt,
             float* out, int* se_rows, float* se_part) {
  const int ho = (h + pt + pb - kh) / sh + 1, wo = (w + pl + pr - kw) / sw + 1;
  const size_t K = (size_t)kh * kw * c, M = (size_t)n * ho * wo;
  std::vector<float> packed((size_t)co * K);
  for (int o = 0; o < co; ++o)
    for (int i = 0; i < c; ++i)
      for (int ky = 0; ky < kh; ++ky)
        for (int kx = 0; kx < kw; ++kx)
          packed[(size_t)o * K + (size_t)(ky * kw + kx) * c + i] = weight[(((size_t)o * c + i) * kh + ky) * kw + kx];
  void* d_in = upload(x, (size_t)n * h * w * c, dt);
  void* d_wt = upload(packed.data(), packed.size(), dt);
  void* d_bias = bias ? upload(bias, co, ppocr::DT_F32) : nullptr;
  void* d_gate = gate ? upload(gate, (size_t)n * c, ppocr::DT_F32) : nullptr;
  void *d_out = nullptr, *d_ws = nullptr, *d_se = nullptr;
  int rc = 0;
  const size_t es = dt == ppocr::DT_BF16 ? 2 : 4;
  if (!d_in || !d_wt || (bias && !d_bias) || (gate && !d_gate) || hipMalloc(&d_out, M * co * es) != hipSuccess ||
      (splits > 1 && hipMalloc(&d_ws, (size_t)splits * M * co * 4) != hipSuccess)) {
    rc = 1;
  } else {
    ppocr::ConvParams p{};
    p.in = d_in;
    p.N = n, p.H = h, p.W = w, p.C = c, p.in_ps = c;
    p.out = d_out;
    p.Ho = ho, p.Wo = wo, p.Co = co, p.out_ps = co;
    p.wt = d_wt;
    p.ldw = (int)K;
    p.bias = static_cast<const float*>(d_bias);
    p.kh = kh, p.kw = kw, p.sh = sh, p.sw = sw, p.pt = pt, p.pl = pl;
    p.act = act;
    p.in_gate = static_cast<const float*>(d_gate);
    p.up_s = 2;
    p.rep = 1;
    p.out_h = ho, p.out_w = wo;
    p.dt = dt;
    p.split_ws = static_cast<float*>(d_ws);
    p.splits = splits;
    if (se_rows) {
      *se_rows = ppocr::conv_se_blocks(p);
      if (*se_rows > 0 && hipMalloc(&d_se, (size_t)*se_rows * co * 4) != hipSuccess) rc = 1;
      p.se_part = static_cast<float*>(d_se);
    }
    if (rc == 0) {
      ppocr::launch_conv(p, nullptr);
      if (hipDeviceSynchronize() != hipSuccess) rc = 1;
    }
    if (rc == 0 && d_se && hipMemcpy(se_part, d_se, (size_t)*se_rows * co * 4, hipMemcpyDeviceToHost) != hipSuccess)
      rc = 1;
    if (rc == 0) {
      if (dt == ppocr::DT_BF16) {
        std::vector<uint16_t> hb(M * co);
        if (hipMemcpy(hb.data(), d_out, hb.size() * 2, hipMemcpyDeviceToHost) != hipSuccess) rc = 1;
        for (size_t i = 0; i < hb.size(); ++i) out[i] = from_bf16(hb[i]);
      } else if (hipMemcpy(out, d_out, M * co * 4, hipMemcpyDeviceToHost) != hipSuccess) {
        rc = 1;
      }
    }
  }
  for (void* ptr : {d_in, d_wt, d_bias, d_gate, d_out, d_ws, d_se})
    if (ptr) (void)hipFree(ptr);
  return rc;
}

// ppocr_probe_depthwise, and with se_rows the SE channel sums the layer
// leaves: *se_rows = depthwise_se_blocks() and se_part [n][*se_rows][c].
int run_depthwise(const float* x, int n, int h, int w, int c, const float* weight, const float* bias, int k, int act,
                  const float* res, int dt, int table, float* out, int* se_rows, float* se_part, int sh = 1,
                  int sw = 1) {
  const size_t px = (size_t)n * h * w;
  const int ho = (h + 2 * (k / 2) - k) / sh + 1, wo = (w + 2 * (k / 2) - k) / sw + 1;
  const size_t opx = (size_t)n * ho * wo;
  std::vector<float> packed((size_t)k * k * c);
  for (int ch = 0; ch < c; ++ch)
    for (int t = 0; t < k * k; ++t) packed[(size_t)t * c + ch] = weight[(size_t)ch * k * k + t];
  void* d_in = upload(x, px * c, dt);
  void* d_wt = upload(packed.data(), packed.size(), ppocr::DT_F32);
  void* d_bias = bias ? upload(bias, c, ppocr::DT_F32) : nullptr;
  void* d_res = res ? upload(res, opx * c, dt) : nullptr;
  void *d_out = nullptr, *d_tab = nullptr, *d_se = nullptr;
  int rc = 0;
  const size_t es = dt == ppocr::DT_BF16 ? 2 : 4;
  if (table) {
    std::vector<uint16_t> tab(ppocr::depthwise_mfma_table_size(c, k));
    ppocr::depthwise_mfma_table(weight, c, k, tab.data());
    if (hipMalloc(&d_tab, tab.size() * 2) != hipSuccess ||
        hipMemcpy(d_tab, tab.data(), tab.size() * 2, hipMemcpyHostToDevice) != hipSuccess)
      rc = 1;
  }
  if (rc || !d_in || !d_wt || (bias && !d_bias) || (res && !d_res) || hipMalloc(&d_out, opx * c * es) != hipSuccess) {
    rc = 1;
  } else {
    ppocr::DwParams p{};
    p.in = d_in;
    p.N = n, p.H = h, p.W = w, p.C = c, p.in_ps = c;
    p.out = d_out;
    p.Ho = ho, p.Wo = wo, p.out_ps = c;
    p.wt = static_cast<const float*>(d_wt);
    p.bias = static_cast<const float*>(d_bias);
    p.kh = p.kw = k, p.sh = sh, p.sw = sw, p.pt = p.pl = k / 2;
    p.act = act;
    p.res = d_res;
    p.res_ps = c;
    p.dt = dt;
    p.wtab = d_tab;
    if (se_rows) {
      *se_rows = ppocr::depthwise_se_blocks(p);
      if (*se_rows == 0) rc = 2;
      else if (hipMalloc(&d_se, (size_t)n * *se_rows * c * 4) != hipSuccess) rc = 1;
      p.se_part = static_cast<float*>(d_se);
    }
    if (rc == 0) ppocr::launch_depthwise(p, nullptr);
    if (rc == 0 && hipDeviceSynchronize() != hipSuccess) rc = 1;
    if (rc == 0 && d_se &&
        hipMemcpy(se_part, d_se, (size_t)n * *se_rows * c * 4, hipMemcpyDeviceToHost) != hipSuccess)
      rc = 1;
    if (rc == 0) {
      if (dt == ppocr::DT_BF16) {
        std::vector<uint16_t> hb(opx * c);
        if (hipMemcpy(hb.data(), d_out, hb.size() * 2, hipMemcpyDeviceToHost) != hipSuccess) rc = 1;
        for (size_t i = 0; i < hb.size(); ++i) out[i] = from_bf16(hb[i]);
      } else if (hipMemcpy(out, d_out, opx * c * 4, hipMemcpyDeviceToHost) != hipSuccess) {
        rc = 1;
      }
    }
  }
  for (void* ptr : {d_in, d_wt, d_bias, d_res, d_out, d_tab, d_se})
    if (ptr) (void)hipFree(ptr);
  return rc;
}

}  // namespace

extern "C" {

// x [n][h][w][c] (c % 4 == 0), weight [co][c][kh][kw], bias [co] (or null),
// gate [n][c] (or null): out [n][ho][wo][co] = act(conv(x * gate) + bias),
// computed with `splits` K splits (1: none) in storage type dt (0 fp32,
// 1 bf16; bf16 output is returned widened).  Returns 0, or 1 on a HIP error.
int ppocr_probe_conv(const float* x, int n, int h, int w, int c, const float* weight, const float* bias, int co,
                     int kh, int kw, int sh, int sw, int pt, int pl, int pb, int pr, int act, const float* gate,
                     int splits, int dt, float* out) {
  return run_conv(x, n, h, w, c, weight, bias, co, kh, kw, sh, sw, pt, pl, pb, pr, act, gate, splits, dt, out,
                  nullptr, nullptr);
}

// ppocr_probe_conv without K splits, also asking for the squeeze-excitation
// channel sums of the output: *rows = conv_se_blocks() (0: the kernel leaves
// none), and se_part [rows][co] (room for ceil(ho*wo/16) + 4 rows, the
// most any tile gives) receives them.
int ppocr_probe_conv_se(const float* x, int h, int w, int c, const float* weight, const float* bias, int co, int kh,
                        int kw, int sh, int sw, int pt, int pl, int pb, int pr, int act, const float* gate, int dt,
                        float* out, int* rows, float* se_part) {
  return run_conv(x, 1, h, w, c, weight, bias, co, kh, kw, sh, sw, pt, pl, pb, pr, act, gate, 1, dt, out, rows,
                  se_part);
}

// 1x1 conv with upsample-on-write (the medium neck's intraclass conv_final):
// x [n][h][w][c], weight [co][c], bias [co], residual res [n][h][w][co] (or
// null): y = res + act(x W^T + b), each pixel written as a rep x rep block
// of out [n][h*rep][w*rep][co]; fp32.  Returns 0, or 1 on a HIP error.
int ppocr_probe_conv_rep(const float* x, int n, int h, int w, int c, const float* weight, const float* bias, int co,
                         int act, const float* res, int rep, float* out) {
  const size_t M = (size_t)n * h * w, O = M * rep * rep * co;
  void* d_in = upload(x, M * c, ppocr::DT_F32);
  void* d_wt = upload(weight, (size_t)co * c, ppocr::DT_F32);
  void* d_bias = upload(bias, co, ppocr::DT_F32);
  void* d_res = res ? upload(res, M * co, ppocr::DT_F32) : nullptr;
  void* d_out = nullptr;
  int rc = 0;
  if (!d_in || !d_wt || !d_bias || (res && !d_res) || hipMalloc(&d_out, O * 4) != hipSuccess) {
    rc = 1;
  } else {
    ppocr::ConvParams p{};
    p.in = d_in;
    p.N = n, p.H = h, p.W = w, p.C = c, p.in_ps = c;
    p.out = d_out;
    p.Ho = h, p.Wo = w, p.Co = co, p.out_ps = co;
    p.wt = d_wt;
    p.ldw = c;
    p.bias = static_cast<const float*>(d_bias);
    p.kh = p.kw = 1, p.sh = p.sw = 1;
    p.act = act;
    p.res = d_res;
    p.res_ps = co;
    p.up_s = 2;
    p.rep = rep;
    p.out_h = h * rep, p.out_w = w * rep;
    p.dt = ppocr::DT_F32;
    p.splits = 1;
    ppocr::launch_conv(p, nullptr);
    if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(out, d_out, O * 4, hipMemcpyDeviceToHost) != hipSuccess)
      rc = 1;
  }
  for (void* ptr : {d_in, d_wt, d_bias, d_res, d_out})
    if (ptr) (void)hipFree(ptr);
  return rc;
}

// 1x1 conv with a residual in storage type dt: x [n][h][w][c], weight
// [co][c], bias [co], res [n][h][w][co] (or null), res_gate [n][co] (or
// null: plain residual): y = res * res_gate + act(x W^T + b), stored in dt,
// or in fp32 with out_f32.  `kernel` (if not null) receives the kernel
// instance's name.  Returns 0, or 1 on a HIP error.
int ppocr_probe_conv1x1_res(const float* x, int n, int h, int w, int c, const float* weight, const float* bias, int co,
                            int act, const float* res, const float* res_gate, int dt, int out_f32, float* out,
                            const char** kernel) {
  static thread_local std::string name;
  const size_t M = (size_t)n * h * w;
  void* d_in = upload(x, M * c, dt);
  void* d_wt = upload(weight, (size_t)co * c, dt);
  void* d_bias = upload(bias, co, ppocr::DT_F32);
  void* d_res = res ? upload(res, M * co, dt) : nullptr;
  void* d_rg = res_gate ? upload(res_gate, (size_t)n * co, ppocr::DT_F32) : nullptr;
  void* d_out = nullptr;
  const size_t es = dt == ppocr::DT_BF16 && !out_f32 ? 2 : 4;
  int rc = 0;
  if (!d_in || !d_wt || !d_bias || (res && !d_res) || (res_gate && !d_rg) ||
      hipMalloc(&d_out, M * co * es) != hipSuccess) {
    rc = 1;
  } else {
    ppocr::ConvParams p{};
    p.in = d_in;
    p.N = n, p.H = h, p.W = w, p.C = c, p.in_ps = c;
    p.out = d_out;
    p.Ho = h, p.Wo = w, p.Co = co, p.out_ps = co;
    p.wt = d_wt;
    p.ldw = c;
    p.bias = static_cast<const float*>(d_bias);
    p.kh = p.kw = 1, p.sh = p.sw = 1;
    p.act = act;
    p.res = d_res;
    p.res_ps = co;
    p.res_gate = static_cast<const float*>(d_rg);
    p.up_s = 2;
    p.rep = 1;
    p.out_h = h, p.out_w = w;
    p.dt = dt;
    p.out_f32 = out_f32 && dt != ppocr::DT_F32;
    p.splits = 1;
    name = ppocr::conv_kernel_name(p);
    if (kernel) *kernel = name.c_str();
    ppocr::launch_conv(p, nullptr);
    if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) rc = 1;
    if (rc == 0) {
      if (es == 2) {
        std::vector<uint16_t> hb(M * co);
        if (hipMemcpy(hb.data(), d_out, hb.size() * 2, hipMemcpyDeviceToHost) != hipSuccess) rc = 1;
        for (size_t i = 0; i < hb.size(); ++i) out[i] = from_bf16(hb[i]);
      } else if (hipMemcpy(out, d_out, M * co * 4, hipMemcpyDeviceToHost) != hipSuccess) {
        rc = 1;
      }
    }
  }
  for (void* ptr : {d_in, d_wt, d_bias, d_res, d_rg, d_out})
    if (ptr) (void)hipFree(ptr);
  return rc;
}

// The kernel instance ppocr_probe_conv runs for these arguments (pointers
// stand in by their alignment: the probe's buffers are hipMalloc'd), and the
// split count the planner would choose for the layer.
const char* ppocr_probe_conv_kernel(int n, int h, int w, int c, int co, int kh, int kw, int sh, int sw, int pt,
                                    int pl, int pb, int pr, int gated, int dt, int* planner_splits) {
  static thread_local std::string name;
  const int ho = (h + pt + pb - kh) / sh + 1, wo = (w + pl + pr - kw) / sw + 1;
  ppocr::ConvParams p{};
  p.N = n, p.H = h, p.W = w, p.C = c, p.in_ps = c;
  p.Ho = ho, p.Wo = wo, p.Co = co, p.out_ps = co;
  p.ldw = kh * kw * c;
  p.kh = kh, p.kw = kw, p.sh = sh, p.sw = sw, p.pt = pt, p.pl = pl;
  p.in_gate = gated ? reinterpret_cast<const float*>((uintptr_t)256) : nullptr;
  p.dt = dt;
  name = ppocr::conv_kernel_name(p);
  if (planner_splits) *planner_splits = ppocr::conv_split_k(n * ho * wo, co, kh * kw * c, dt);
  return name.c_str();
}

// Depthwise: x [n][h][w][c] (c % 4 == 0), weight [c][k][k], bias [c] (or
// null), residual [n][ho][wo][c] (or null): out = res + act(dw(x) + bias)
// with stride 1 and pads (k / 2 each side), in storage type dt; table != 0
// also packs the matrix-core tap fragments, as a bf16 plan does.  Returns 0,
// or 1 on a HIP error.
int ppocr_probe_depthwise(const float* x, int n, int h, int w, int c, const float* weight, const float* bias, int k,
                          int act, const float* res, int dt, int table, float* out) {
  return run_depthwise(x, n, h, w, c, weight, bias, k, act, res, dt, table, out, nullptr, nullptr);
}

// A 3x3 depthwise (pads 1, no residual, no table) with strides (sh, sw):
// out [n][(h - 1) / sh + 1][(w - 1) / sw + 1][c].  Returns 0, or 1 on a HIP
// error.
int ppocr_probe_depthwise_strided(const float* x, int n, int h, int w, int c, const float* weight, const float* bias,
                                  int sh, int sw, int act, int dt, float* out) {
  return run_depthwise(x, n, h, w, c, weight, bias, 3, act, nullptr, dt, 0, out, nullptr, nullptr, sh, sw);
}

// The kernel instance ppocr_probe_depthwise_strided runs.
const char* ppocr_probe_depthwise_strided_kernel(int h, int c, int sh, int sw, int dt) {
  return ppocr::depthwise_kernel_name(3, 3, sh, sw, (h - 1) / sh + 1, dt, false, c);
}

// ppocr_probe_depthwise (no residual, no table) also leaving the SE channel
// sums of its stored output: *rows = depthwise_se_blocks() partial rows per
// image and se_part [n][*rows][c] (room for n * ceil(h / 4) * ceil(w / 8)
// rows).  Returns 0, 1 on a HIP error, 2 when the layer leaves no sums.
int ppocr_probe_depthwise_se(const float* x, int n, int h, int w, int c, const float* weight, const float* bias,
                             int act, int dt, float* out, int* rows, float* se_part) {
  return run_depthwise(x, n, h, w, c, weight, bias, 3, act, nullptr, dt, 0, out, rows, se_part);
}

// Depthwise with the gate-residual prologue (fp32): x = h + h * gate[n]
// (+ the nearest 2x upsample of up [n][h/2][w/2][c], or null) is the input
// of a k x k stride-1 depthwise (pads k / 2, bias, no activation); out [n][h][w][c]
// is the conv, xout [n][h][w][c] (or null) receives x.  Returns 0, or 1 on a
// HIP error.
int ppocr_probe_depthwise_gate_residual(const float* h, int n, int ht, int wd, int c, const float* gate,
                                        const float* up, const float* weight, const float* bias, int k, float* out,
                                        float* xout) {
  const size_t px = (size_t)n * ht * wd;
  std::vector<float> packed((size_t)k * k * c);
  for (int ch = 0; ch < c; ++ch)
    for (int t = 0; t < k * k; ++t) packed[(size_t)t * c + ch] = weight[(size_t)ch * k * k + t];
  void* d_in = upload(h, px * c, ppocr::DT_F32);
  void* d_gate = upload(gate, (size_t)n * c, ppocr::DT_F32);
  void* d_up = up ? upload(up, (size_t)n * (ht / 2) * (wd / 2) * c, ppocr::DT_F32) : nullptr;
  void* d_wt = upload(packed.data(), packed.size(), ppocr::DT_F32);
  void* d_bias = upload(bias, c, ppocr::DT_F32);
  void *d_out = nullptr, *d_x = nullptr;
  int rc = 0;
  if (!d_in || !d_gate || (up && !d_up) || !d_wt || !d_bias || hipMalloc(&d_out, px * c * 4) != hipSuccess ||
      (xout && hipMalloc(&d_x, px * c * 4) != hipSuccess) || !ppocr::depthwise_gate_residual_supported(k, k, 1, 1) ||
      (up && (ht % 2 || wd % 2))) {
    rc = 1;
  } else {
    ppocr::DwParams p{};
    p.in = d_in;
    p.N = n, p.H = ht, p.W = wd, p.C = c, p.in_ps = c;
    p.out = d_out;
    p.Ho = ht, p.Wo = wd, p.out_ps = c;
    p.wt = static_cast<const float*>(d_wt);
    p.bias = static_cast<const float*>(d_bias);
    p.kh = p.kw = k, p.sh = p.sw = 1, p.pt = p.pl = k / 2;
    p.act = 0;
    p.dt = ppocr::DT_F32;
    p.gr_gate = static_cast<const float*>(d_gate);
    p.gr_up = d_up;
    p.gr_up_ps = c;
    p.gr_out = d_x;
    p.gr_out_ps = c;
    ppocr::launch_depthwise(p, nullptr);
    if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(out, d_out, px * c * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        (xout && hipMemcpy(xout, d_x, px * c * 4, hipMemcpyDeviceToHost) != hipSuccess))
      rc = 1;
  }
  for (void* ptr : {d_in, d_gate, d_up, d_wt, d_bias, d_out, d_x})
    if (ptr) (void)hipFree(ptr);
  return rc;
}

// The matrix-core tap fragments a bf16 plan packs for a c-channel k x k
// depthwise layer (host only): taps [c][k][k] -> out [c][k][64][8] bf16 bits.
void ppocr_probe_depthwise_table(const float* weight, int c, int k, uint16_t* out) {
  ppocr::depthwise_mfma_table(weight, c, k, out);
}

// Fused pointwise pair (pair_gemm.hip) on host arrays: x [m][c] rows
// (pixels of n images of hw pixels each), gate [n][c] or null, w1 [h2][c],
// b1 [h2], w2 [co][h2], b2 [co]; out [m][co] = w2 GELU(w1 x' + b1) + b2
// (+ x' when residual), x' = x * gate.  Returns 0, or 1 on a HIP error.
int ppocr_probe_pointwise_pair(const float* x, int m, int hw, int c, const float* gate, const float* w1,
                               const float* b1, int h2, const float* w2, const float* b2, int co, int residual,
                               float* out) {
  const int n = (m + hw - 1) / hw;
  void* d_in = upload(x, (size_t)m * c, ppocr::DT_F32);
  void* d_gate = gate ? upload(gate, (size_t)n * c, ppocr::DT_F32) : nullptr;
  void* d_w1 = upload(w1, (size_t)h2 * c, ppocr::DT_F32);
  void* d_b1 = upload(b1, h2, ppocr::DT_F32);
  void* d_w2 = upload(w2, (size_t)co * h2, ppocr::DT_F32);
  void* d_b2 = upload(b2, co, ppocr::DT_F32);
  void* d_out = nullptr;
  int rc = 0;
  if (!d_in || (gate && !d_gate) || !d_w1 || !d_b1 || !d_w2 || !d_b2 ||
      hipMalloc(&d_out, (size_t)m * co * 4) != hipSuccess || !ppocr::pointwise_pair_supported(c, h2, co, 0)) {
    rc = 1;
  } else {
    ppocr::PairParams p{};
    p.in = static_cast<const float*>(d_in);
    p.in_ps = c;
    p.gate = static_cast<const float*>(d_gate);
    p.HW = hw;
    p.M = m, p.C = c, p.H2 = h2, p.Co = co;
    p.w1 = static_cast<const float*>(d_w1), p.ldw1 = c, p.b1 = static_cast<const float*>(d_b1);
    p.w2 = static_cast<const float*>(d_w2), p.ldw2 = h2, p.b2 = static_cast<const float*>(d_b2);
    p.residual = residual;
    p.out = static_cast<float*>(d_out);
    p.out_ps = co;
    ppocr::launch_pointwise_pair(p, nullptr);
    if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(out, d_out, (size_t)m * co * 4, hipMemcpyDeviceToHost) != hipSuccess)
      rc = 1;
  }
  for (void* d : {d_in, d_gate, d_w1, d_b1, d_w2, d_b2, d_out})
    if (d) (void)hipFree(d);
  return rc;
}

// ppocr_probe_pointwise_pair for one image (m pixels) whose SE gate the
// kernel forms itself: part [P][c] partial channel sums of x, se_w1 [cr][c],
// se_b1 [cr], se_w2 [c][cr], se_b2 [c], gate act(W2 relu(W1 sum/m + b1) +
// b2) with activation se_act.  Returns 0, 1 on a HIP error, 2 when the
// shape is outside pair_se_fold_supported.
int ppocr_probe_pointwise_pair_se(const float* x, int m, int c, const float* part, int P, const float* se_w1,
                                  const float* se_b1, int cr, const float* se_w2, const float* se_b2, int se_act,
                                  const float* w1, const float* b1, int h2, const float* w2, const float* b2, int co,
                                  int residual, float* out) {
  if (!ppocr::pair_se_fold_supported(1, c, h2, cr, P)) return 2;
  void* d_in = upload(x, (size_t)m * c, ppocr::DT_F32);
  void* d_part = upload(part, (size_t)P * c, ppocr::DT_F32);
  void* d_sw1 = upload(se_w1, (size_t)cr * c, ppocr::DT_F32);
  void* d_sb1 = upload(se_b1, cr, ppocr::DT_F32);
  void* d_sw2 = upload(se_w2, (size_t)c * cr, ppocr::DT_F32);
  void* d_sb2 = upload(se_b2, c, ppocr::DT_F32);
  void* d_w1 = upload(w1, (size_t)h2 * c, ppocr::DT_F32);
  void* d_b1 = upload(b1, h2, ppocr::DT_F32);
  void* d_w2 = upload(w2, (size_t)co * h2, ppocr::DT_F32);
  void* d_b2 = upload(b2, co, ppocr::DT_F32);
  void* d_out = nullptr;
  int rc = 0;
  if (!d_in || !d_part || !d_sw1 || !d_sb1 || !d_sw2 || !d_sb2 || !d_w1 || !d_b1 || !d_w2 || !d_b2 ||
      hipMalloc(&d_out, (size_t)m * co * 4) != hipSuccess || !ppocr::pointwise_pair_supported(c, h2, co, 0)) {
    rc = 1;
  } else {
    ppocr::PairParams p{};
    p.in = static_cast<const float*>(d_in);
    p.in_ps = c;
    p.HW = m;
    p.M = m, p.C = c, p.H2 = h2, p.Co = co;
    p.w1 = static_cast<const float*>(d_w1), p.ldw1 = c, p.b1 = static_cast<const float*>(d_b1);
    p.w2 = static_cast<const float*>(d_w2), p.ldw2 = h2, p.b2 = static_cast<const float*>(d_b2);
    p.residual = residual;
    p.out = static_cast<float*>(d_out);
    p.out_ps = co;
    p.se_part = static_cast<const float*>(d_part);
    p.se_P = P, p.se_Cr = cr, p.se_act = se_act;
    p.se_w1 = static_cast<const float*>(d_sw1), p.se_b1 = static_cast<const float*>(d_sb1);
    p.se_w2 = static_cast<const float*>(d_sw2), p.se_b2 = static_cast<const float*>(d_sb2);
    ppocr::launch_pointwise_pair(p, nullptr);
    if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(out, d_out, (size_t)m * co * 4, hipMemcpyDeviceToHost) != hipSuccess)
      rc = 1;
  }
  for (void* d : {d_in, d_part, d_sw1, d_sb1, d_sw2, d_sb2, d_w1, d_b1, d_w2, d_b2, d_out})
    if (d) (void)hipFree(d);
  return rc;
}

// Fused 3x3 depthwise -> pointwise pair (the pair kernel's depthwise
// prologue) on host arrays: x [n][h][w][c], dw [9][c] taps, dwb [c], stride
// (sh, sw), pads 1; then as ppocr_probe_pointwise_pair on the depthwise
// output (never stored) without a gate; out [n][ho][wo][co].  Returns 0, or
// 1 on a HIP error.
int ppocr_probe_pointwise_pair_dw(const float* x, int n, int h, int w, int c, const float* dw, const float* dwb,
                                  int sh, int sw, const float* w1, const float* b1, int h2, const float* w2,
                                  const float* b2, int co, int residual, float* out) {
  const int ho = (h + 2 - 3) / sh + 1, wo = (w + 2 - 3) / sw + 1;
  const size_t m = (size_t)n * ho * wo;
  void* d_in = upload(x, (size_t)n * h * w * c, ppocr::DT_F32);
  void* d_dw = upload(dw, (size_t)9 * c, ppocr::DT_F32);
  void* d_dwb = upload(dwb, c, ppocr::DT_F32);
  void* d_w1 = upload(w1, (size_t)h2 * c, ppocr::DT_F32);
  void* d_b1 = upload(b1, h2, ppocr::DT_F32);
  void* d_w2 = upload(w2, (size_t)co * h2, ppocr::DT_F32);
  void* d_b2 = upload(b2, co, ppocr::DT_F32);
  void* d_out = nullptr;
  int rc = 0;
  if (!d_in || !d_dw || !d_dwb || !d_w1 || !d_b1 || !d_w2 || !d_b2 || hipMalloc(&d_out, m * co * 4) != hipSuccess ||
      !ppocr::pointwise_pair_supported(c, h2, co, 0)) {
    rc = 1;
  } else {
    ppocr::PairParams p{};
    p.HW = ho * wo;
    p.M = (int)m, p.C = c, p.H2 = h2, p.Co = co;
    p.w1 = static_cast<const float*>(d_w1), p.ldw1 = c, p.b1 = static_cast<const float*>(d_b1);
    p.w2 = static_cast<const float*>(d_w2), p.ldw2 = h2, p.b2 = static_cast<const float*>(d_b2);
    p.residual = residual;
    p.out = static_cast<float*>(d_out);
    p.out_ps = co;
    p.dw_in = static_cast<const float*>(d_in);
    p.dw_ps = c, p.dw_h = h, p.dw_w = w, p.dw_wo = wo, p.dw_sh = sh, p.dw_sw = sw, p.dw_pt = 1, p.dw_pl = 1;
    p.dw_wt = static_cast<const float*>(d_dw);
    p.dw_b = static_cast<const float*>(d_dwb);
    ppocr::launch_pointwise_pair(p, nullptr);
    if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(out, d_out, m * co * 4, hipMemcpyDeviceToHost) != hipSuccess)
      rc = 1;
  }
  for (void* d : {d_in, d_dw, d_dwb, d_w1, d_b1, d_w2, d_b2, d_out})
    if (d) (void)hipFree(d);
  return rc;
}

// The bf16 pointwise pair on host arrays, twice: fused (launch_pair_bf16)
// into out_fused, and as the unfused bf16 plan runs it (the gate pass
// storing x * g, then channel_conv1 and channel_conv2 on the direct conv
// kernel with the stored x * g as residual) into out_unfused.  x [m][c]
// (hw pixels per image), gate [m / hw][c] or null, w1 [2c][c], b1 [2c],
// w2 [c][2c], b2 [c]; x and the weights are rounded to bf16, the outputs
// [m][c] are returned widened.  *kernel (cap bytes) receives the fused
// kernel's instance name.  Returns 0, 1 on a HIP error, 2 for a shape the
// fused kernel does not take.
int ppocr_probe_pair_bf16(const float* x, int m, int hw, int c, const float* gate, const float* w1, const float* b1,
                          const float* w2, const float* b2, int residual, float* out_fused, float* out_unfused,
                          char* kernel, size_t cap) {
  if (!ppocr::pair_bf16_supported(c, 2 * c, c) || m <= 0 || hw <= 0) return 2;
  const int n = (m + hw - 1) / hw;
  const int BF = ppocr::DT_BF16, F = ppocr::DT_F32;
  // The gate pass covers whole images (n * hw rows): x and x * g are
  // allocated that long, x zero past row m.
  const size_t rows = (size_t)n * hw;
  std::vector<float> xpad(rows * c, 0.0f);
  memcpy(xpad.data(), x, (size_t)m * c * sizeof(float));
  void* d_in = upload(xpad.data(), rows * c, BF);
  void* d_gate = gate ? upload(gate, (size_t)n * c, F) : nullptr;
  void* d_w1 = upload(w1, (size_t)2 * c * c, BF);
  void* d_b1 = upload(b1, 2 * c, F);
  void* d_w2 = upload(w2, (size_t)2 * c * c, BF);
  void* d_b2 = upload(b2, c, F);
  void *d_xs = nullptr, *d_h = nullptr, *d_o1 = nullptr, *d_o2 = nullptr;
  int rc = 0;
  if (!d_in || (gate && !d_gate) || !d_w1 || !d_b1 || !d_w2 || !d_b2 || hipMalloc(&d_xs, rows * c * 2) ||
      hipMalloc(&d_h, (size_t)m * 2 * c * 2) || hipMalloc(&d_o1, (size_t)m * c * 2) ||
      hipMalloc(&d_o2, (size_t)m * c * 2)) {
    rc = 1;
  } else {
    ppocr::PairBf16Params p{};
    p.in = d_in, p.in_ps = c;
    p.gate = static_cast<const float*>(d_gate), p.HW = hw;
    p.M = m, p.C = c;
    p.w1 = d_w1, p.ldw1 = c, p.b1 = static_cast<const float*>(d_b1);
    p.w2 = d_w2, p.ldw2 = 2 * c, p.b2 = static_cast<const float*>(d_b2);
    p.residual = residual;
    p.out = d_o1, p.out_ps = c;
    if (kernel && cap) {
      const std::string name = ppocr::pair_bf16_kernel_name(p);
      const size_t k = std::min(cap - 1, name.size());
      memcpy(kernel, name.data(), k);
      kernel[k] = 0;
    }
    ppocr::launch_pair_bf16(p, nullptr);
    if (hipGetLastError() != hipSuccess) rc = 1;
    // Unfused: x * g stored, conv1 (GELU), conv2 (+ residual).
    const void* a = d_in;
    if (gate) {
      ppocr::launch_scale_channels(d_in, n, hw, c, c, static_cast<const float*>(d_gate), d_xs, BF, nullptr);
      a = d_xs;
    }
    ppocr::ConvParams q{};
    q.N = 1, q.H = m, q.W = 1, q.Ho = m, q.Wo = 1, q.out_h = m, q.out_w = 1;
    q.kh = q.kw = q.sh = q.sw = 1;
    q.up_s = 2, q.rep = 1, q.dt = BF, q.splits = 1;
    ppocr::ConvParams q1 = q, q2 = q;
    q1.in = a, q1.C = q1.in_ps = c, q1.wt = d_w1, q1.ldw = c, q1.bias = static_cast<const float*>(d_b1);
    q1.Co = q1.out_ps = 2 * c, q1.act = ppocr::ACT_GELU, q1.out = d_h;
    q2.in = d_h, q2.C = q2.in_ps = 2 * c, q2.wt = d_w2, q2.ldw = 2 * c, q2.bias = static_cast<const float*>(d_b2);
    q2.Co = q2.out_ps = c, q2.out = d_o2;
    if (residual) q2.res = a, q2.res_ps = c;
    if (ppocr::conv_split_k(m, 2 * c, c, BF) > 1 || ppocr::conv_split_k(m, c, 2 * c, BF) > 1) rc = 2;
    if (rc == 0) {
      ppocr::launch_conv(q1, nullptr);
      ppocr::launch_conv(q2, nullptr);
      if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) rc = 1;
    }
    std::vector<uint16_t> hb((size_t)m * c);
    for (auto [d, o] : {std::pair<void*, float*>{d_o1, out_fused}, {d_o2, out_unfused}}) {
      if (rc != 0) break;
      if (hipMemcpy(hb.data(), d, hb.size() * 2, hipMemcpyDeviceToHost) != hipSuccess) rc = 1;
      for (size_t i = 0; i < hb.size(); ++i) o[i] = from_bf16(hb[i]);
    }
  }
  for (void* d : {d_in, d_gate, d_w1, d_b1, d_w2, d_b2, d_xs, d_h, d_o1, d_o2})
    if (d) (void)hipFree(d);
  return rc;
}

// The kernel instance ppocr_probe_depthwise runs.
const char* ppocr_probe_depthwise_kernel(int h, int c, int k, int dt, int table) {
  return ppocr::depthwise_kernel_name(k, k, 1, 1, h, dt, table != 0, c);
}

// Batched FPN gates on host arrays.  Gate i (dims[4i..4i+3] = HW, C, P, Cr)
// takes its partial sums [n][P][C], w1 [Cr][C], b1 [Cr], w2 [C][Cr], b2 [C]
// from the concatenation of the per-gate arrays, in gate order; gates [n][C]
// are written the same way.  Returns 0, 1 on a HIP error, 2 when the gates
// cannot share one launch.
int ppocr_probe_se_multi(int count, int n, const int* dims, const float* part, const float* w1, const float* b1,
                         const float* w2, const float* b2, int act, float* gates) {
  if (count < 1 || count > ppocr::kSeMultiMax) return 2;
  ppocr::SeMulti m{};
  m.count = count;
  std::vector<void*> bufs;
  size_t op = 0, ow1 = 0, ob1 = 0, ow2 = 0, ob2 = 0, og = 0;
  int rc = 0;
  int kind = -1;
  for (int i = 0; i < count && rc == 0; ++i) {
    const int HW = dims[4 * i], C = dims[4 * i + 1], P = dims[4 * i + 2], Cr = dims[4 * i + 3];
    ppocr::SeParams q{};
    q.N = n, q.HW = HW, q.C = C, q.in_ps = C, q.P = P, q.Cr = Cr, q.gate_act = act, q.dt = ppocr::DT_F32;
    const int k = ppocr::se_multi_kind(q);
    if (k == 0 || (kind >= 0 && k != kind)) rc = 2;
    kind = k;
    void* d[6] = {upload(part + op, (size_t)n * P * C, ppocr::DT_F32), upload(w1 + ow1, (size_t)Cr * C, ppocr::DT_F32),
                  upload(b1 + ob1, Cr, ppocr::DT_F32),                upload(w2 + ow2, (size_t)C * Cr, ppocr::DT_F32),
                  upload(b2 + ob2, C, ppocr::DT_F32),                 nullptr};
    if (hipMalloc(&d[5], (size_t)n * C * 4) != hipSuccess) d[5] = nullptr;
    for (void* b : d) {
      bufs.push_back(b);
      if (!b) rc = rc ? rc : 1;
    }
    q.partial = static_cast<float*>(d[0]);
    q.w1 = static_cast<const float*>(d[1]), q.b1 = static_cast<const float*>(d[2]);
    q.w2 = static_cast<const float*>(d[3]), q.b2 = static_cast<const float*>(d[4]);
    q.gate = static_cast<float*>(d[5]);
    m.p[i] = q;
    op += (size_t)n * P * C, ow1 += (size_t)Cr * C, ob1 += Cr, ow2 += (size_t)C * Cr, ob2 += C;
  }
  if (rc == 0) {
    ppocr::launch_se_multi(m, nullptr);
    if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) rc = 1;
    for (int i = 0; i < count && rc == 0; ++i) {
      const size_t bytes = (size_t)n * m.p[i].C * 4;
      if (hipMemcpy(gates + og, m.p[i].gate, bytes, hipMemcpyDeviceToHost) != hipSuccess) rc = 1;
      og += (size_t)n * m.p[i].C;
    }
  }
  for (void* b : bufs)
    if (b) (void)hipFree(b);
  return rc;
}

// Batched gate_residual writes on host arrays: part i (dims[4i..4i+3] = H,
// W, C, rep) reads x [n][H][W][C] and gate [n][C] and writes out
// [n][H rep][W rep][C], each array the concatenation of the per-part ones.
// Returns 0, or 1 on a HIP error.
int ppocr_probe_gate_residual_multi(int count, int n, const int* dims, const float* x, const float* gate,
                                    float* out) {
  if (count < 1 || count > 4) return 1;
  ppocr::GateResidualMulti m{};
  m.count = count, m.N = n, m.dt = ppocr::DT_F32;
  std::vector<void*> bufs;
  size_t ox = 0, og = 0;
  int rc = 0;
  for (int i = 0; i < count; ++i) {
    const int H = dims[4 * i], W = dims[4 * i + 1], C = dims[4 * i + 2], rep = dims[4 * i + 3];
    void* dx = upload(x + ox, (size_t)n * H * W * C, ppocr::DT_F32);
    void* dg = upload(gate + og, (size_t)n * C, ppocr::DT_F32);
    void* dout = nullptr;
    if (hipMalloc(&dout, (size_t)n * H * rep * W * rep * C * 4) != hipSuccess) dout = nullptr;
    for (void* b : {dx, dg, dout}) {
      bufs.push_back(b);
      if (!b) rc = 1;
    }
    m.part[i] = ppocr::GateResidualPart{dx, H, W, C, C, static_cast<const float*>(dg), dout, C, rep};
    ox += (size_t)n * H * W * C, og += (size_t)n * C;
  }
  if (rc == 0) {
    ppocr::launch_gate_residual_multi(m, nullptr);
    if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) rc = 1;
    size_t oo = 0;
    for (int i = 0; i < count && rc == 0; ++i) {
      const ppocr::GateResidualPart& q = m.part[i];
      const size_t cnt = (size_t)n * q.H * q.rep * q.W * q.rep * q.C;
      if (hipMemcpy(out + oo, q.out, cnt * 4, hipMemcpyDeviceToHost) != hipSuccess) rc = 1;
      oo += cnt;
    }
  }
  for (void* b : bufs)
    if (b) (void)hipFree(b);
  return rc;
}


// The bf16 rounding points of a model's bf16 plan (plan_rounding_points),
// built on the host from a safetensors file (no device work): one per line,
// "A <value>" or "W <layer>", into `out` (NUL terminated, cut at `cap`).
// kind 0 detector, 1 recognizer.  Returns the bytes needed (with the
// terminator), or -1 on an error.
long ppocr_probe_plan_rounding(const char* path, int kind, int size, int n, int h, int w, char* out, size_t cap) {
  try {
    ppocr::SafeTensors st = ppocr::SafeTensors::load(path);
    const size_t nchw[4] = {(size_t)n, 3, (size_t)h, (size_t)w};
    ppocr::Plan plan = kind == 0 ? ppocr::build_detector(st, size, nchw, ppocr::DT_BF16)
                                 : ppocr::build_recognizer(st, size, nchw, ppocr::DT_BF16, false);
    std::string text;
    for (const std::string& r : ppocr::plan_rounding_points(plan)) text += r + "\n";
    if (out && cap) {
      const size_t k = std::min(cap - 1, text.size());
      memcpy(out, text.data(), k);
      out[k] = 0;
    }
    return (long)text.size() + 1;
  } catch (...) {
    return -1;
  }
}

}  // extern "C"
