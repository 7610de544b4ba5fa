// Bandwidth-bound kernels of the detector and recognizer: depthwise conv,
// squeeze-excitation, FPN gate/upsample/concat, pools, the fused DB head
// tail, LayerNorm, attention, row softmax and image preprocessing.
//
// All activations are NHWC with C % 4 == 0, so one lane moves one float4
// (16 B) along the channel axis and consecutive lanes touch consecutive
// 16 B segments: every global access of these kernels is fully coalesced.
#include "device_math.h"

namespace ppocr {

static inline unsigned blocks_for(long n, int per = 256) { return (unsigned)((n + per - 1) / per); }

// ----------------------------------------------------------------- depthwise
// Replaces WGSL `depthwise` (src/gpu/shaders/depthwise.wgsl:77); semantics of
// the reference CPU depthwise (src/cpu/ops.rs:385-826): zero padding, bias,
// activation, then optional residual add (x + act(dw(x) + b)).
__global__ __launch_bounds__(256) void depthwise_kernel(DwParams p) {
  const int C4 = p.C >> 2;
  long idx = (long)blockIdx.x * 256 + threadIdx.x;
  long total = (long)p.N * p.Ho * p.Wo * C4;
  if (idx >= total) return;
  int c4 = (int)(idx % C4);
  long pix = idx / C4;
  int ox = (int)(pix % p.Wo);
  long t = pix / p.Wo;
  int oy = (int)(t % p.Ho);
  int n = (int)(t / p.Ho);
  const int c = c4 * 4;
  float4 acc = f4_zero();
  for (int ky = 0; ky < p.kh; ++ky) {
    int iy = oy * p.sh - p.pt + ky;
    if (iy < 0 || iy >= p.H) continue;
    const float* row = p.in + (size_t)(n * p.H + iy) * p.W * p.in_ps + c;
    const float* wrow = p.wt + (size_t)ky * p.kw * p.C + c;
    for (int kx = 0; kx < p.kw; ++kx) {
      int ix = ox * p.sw - p.pl + kx;
      if (ix < 0 || ix >= p.W) continue;
      float4 x = *reinterpret_cast<const float4*>(row + (size_t)ix * p.in_ps);
      float4 w = *reinterpret_cast<const float4*>(wrow + (size_t)kx * p.C);
      acc.x = fmaf(x.x, w.x, acc.x);
      acc.y = fmaf(x.y, w.y, acc.y);
      acc.z = fmaf(x.z, w.z, acc.z);
      acc.w = fmaf(x.w, w.w, acc.w);
    }
  }
  if (p.bias) {
    float4 b = *reinterpret_cast<const float4*>(p.bias + c);
    acc.x += b.x;
    acc.y += b.y;
    acc.z += b.z;
    acc.w += b.w;
  }
  acc.x = act_apply(p.act, acc.x);
  acc.y = act_apply(p.act, acc.y);
  acc.z = act_apply(p.act, acc.z);
  acc.w = act_apply(p.act, acc.w);
  if (p.res) {
    float4 r = *reinterpret_cast<const float4*>(p.res + (size_t)pix * p.res_ps + c);
    acc.x = r.x + acc.x;
    acc.y = r.y + acc.y;
    acc.z = r.z + acc.z;
    acc.w = r.w + acc.w;
  }
  *reinterpret_cast<float4*>(p.out + (size_t)pix * p.out_ps + c) = acc;
}

void launch_depthwise(const DwParams& p, hipStream_t s) {
  long total = (long)p.N * p.Ho * p.Wo * (p.C / 4);
  hipLaunchKernelGGL(depthwise_kernel, dim3(blocks_for(total)), dim3(256), 0, s, p);
}

// ----------------------------------------------------------------- SE gate
// Replaces WGSL `global_mean` + two `conv_single_row` + activation
// (src/gpu/shaders/pool.wgsl:183, conv_single_row.wgsl:84).  Stage 1: each
// block sums a chunk of pixels for all channels (lanes split channels x
// pixel phases, fixed-order LDS reduction).  Stage 2: one block per image
// finishes the mean and runs both 1x1 convs of the squeeze-excitation.
__global__ __launch_bounds__(256) void se_partial_kernel(SeParams p, int chunk) {
  __shared__ float4 red[256];
  const int C4 = p.C >> 2;
  const int lanes_p = 256 / C4;
  const int tid = threadIdx.x;
  const int cq = tid % C4;
  const int pl = tid / C4;
  const int n = blockIdx.y;
  const int start = blockIdx.x * chunk;
  const int end = min(start + chunk, p.HW);
  float4 s = f4_zero();
  if (pl < lanes_p) {
    const float* base = p.in + (size_t)n * p.HW * p.in_ps + cq * 4;
    for (int px = start + pl; px < end; px += lanes_p) {
      float4 v = *reinterpret_cast<const float4*>(base + (size_t)px * p.in_ps);
      s.x += v.x;
      s.y += v.y;
      s.z += v.z;
      s.w += v.w;
    }
  }
  red[tid] = s;
  __syncthreads();
  if (tid < C4) {
    float4 t = red[tid];
    for (int k = 1; k < lanes_p; ++k) {
      float4 v = red[k * C4 + tid];
      t.x += v.x;
      t.y += v.y;
      t.z += v.z;
      t.w += v.w;
    }
    *reinterpret_cast<float4*>(p.partial + ((size_t)n * p.P + blockIdx.x) * p.C + tid * 4) = t;
  }
}

__global__ __launch_bounds__(256) void se_gate_kernel(SeParams p) {
  extern __shared__ float sm[];
  float* mean = sm;           // [C]
  float* hidden = sm + p.C;   // [Cr]
  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  for (int c = tid; c < p.C; c += 256) {
    float s = 0.0f;
    for (int k = 0; k < p.P; ++k) s += p.partial[((size_t)n * p.P + k) * p.C + c];
    mean[c] = s / (float)p.HW;
  }
  __syncthreads();
  for (int j = tid; j < p.Cr; j += 256) {
    const float* w = p.w1 + (size_t)j * p.C;
    float acc = 0.0f;
    for (int c = 0; c < p.C; ++c) acc = fmaf(w[c], mean[c], acc);
    hidden[j] = fmaxf(acc + p.b1[j], 0.0f);
  }
  __syncthreads();
  for (int c = tid; c < p.C; c += 256) {
    const float* w = p.w2 + (size_t)c * p.Cr;
    float acc = 0.0f;
    for (int j = 0; j < p.Cr; ++j) acc = fmaf(w[j], hidden[j], acc);
    p.gate[(size_t)n * p.C + c] = act_apply(p.gate_act, acc + p.b2[c]);
  }
}

void launch_se(const SeParams& p, hipStream_t s) {
  int chunk = (p.HW + p.P - 1) / p.P;
  hipLaunchKernelGGL(se_partial_kernel, dim3(p.P, p.N), dim3(256), 0, s, p, chunk);
  size_t lds = (size_t)(p.C + p.Cr) * sizeof(float);
  hipLaunchKernelGGL(se_gate_kernel, dim3(p.N), dim3(256), lds, s, p);
}

// ----------------------------------------------------------------- layout
__global__ void nchw_to_nhwc4_kernel(const float* in, float* out, int N, int H, int W) {
  long idx = (long)blockIdx.x * 256 + threadIdx.x;
  long plane = (long)H * W;
  if (idx >= (long)N * plane) return;
  int n = (int)(idx / plane);
  long i = idx - n * plane;
  const float* src = in + (size_t)n * 3 * plane + i;
  *reinterpret_cast<float4*>(out + (size_t)idx * 4) = make_float4(src[0], src[plane], src[2 * plane], 0.0f);
}

void launch_nchw_to_nhwc4(const float* in, float* out, int N, int H, int W, hipStream_t s) {
  hipLaunchKernelGGL(nchw_to_nhwc4_kernel, dim3(blocks_for((long)N * H * W)), dim3(256), 0, s, in, out, N, H, W);
}

// ----------------------------------------------------------------- pools
// Max pool 2x2 / stride 1 / pads (0,0,1,1) of the large stem
// (src/cpu/model.rs:689, src/cpu/ops.rs:1520-1535); fmaxf ignores NaN like
// f32::max.
__global__ void maxpool_same_kernel(const float* in, int N, int H, int W, int C, int in_ps, float* out, int out_ps) {
  const int C4 = C >> 2;
  long idx = (long)blockIdx.x * 256 + threadIdx.x;
  long total = (long)N * H * W * C4;
  if (idx >= total) return;
  int c = (int)(idx % C4) * 4;
  long pix = idx / C4;
  int x = (int)(pix % W);
  long t = pix / W;
  int y = (int)(t % H);
  int n = (int)(t / H);
  float4 m = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
  for (int dy = 0; dy < 2; ++dy)
    for (int dx = 0; dx < 2; ++dx) {
      int iy = y + dy, ix = x + dx;
      if (iy >= H || ix >= W) continue;
      float4 v = *reinterpret_cast<const float4*>(in + ((size_t)(n * H + iy) * W + ix) * in_ps + c);
      m.x = fmaxf(m.x, v.x);
      m.y = fmaxf(m.y, v.y);
      m.z = fmaxf(m.z, v.z);
      m.w = fmaxf(m.w, v.w);
    }
  *reinterpret_cast<float4*>(out + (size_t)pix * out_ps + c) = m;
}

void launch_maxpool_same(const float* in, int N, int H, int W, int C, int in_ps, float* out, int out_ps,
                         hipStream_t s) {
  long total = (long)N * H * W * (C / 4);
  hipLaunchKernelGGL(maxpool_same_kernel, dim3(blocks_for(total)), dim3(256), 0, s, in, N, H, W, C, in_ps, out,
                     out_ps);
}

// Average pool [3,2] / [3,2], no padding, count_include_pad = false
// (src/cpu/ops.rs:1537-1604): the six taps are summed in row-major order.
__global__ void avgpool32_kernel(const float* in, int N, int H, int W, int C, int in_ps, float* out, int Ho,
                                 int Wo) {
  const int C4 = C >> 2;
  long idx = (long)blockIdx.x * 256 + threadIdx.x;
  long total = (long)N * Ho * Wo * C4;
  if (idx >= total) return;
  int c = (int)(idx % C4) * 4;
  long pix = idx / C4;
  int ox = (int)(pix % Wo);
  long t = pix / Wo;
  int oy = (int)(t % Ho);
  int n = (int)(t / Ho);
  float4 s = f4_zero();
  for (int ky = 0; ky < 3; ++ky)
    for (int kx = 0; kx < 2; ++kx) {
      float4 v =
          *reinterpret_cast<const float4*>(in + ((size_t)(n * H + oy * 3 + ky) * W + ox * 2 + kx) * in_ps + c);
      s.x = s.x + v.x;
      s.y = s.y + v.y;
      s.z = s.z + v.z;
      s.w = s.w + v.w;
    }
  *reinterpret_cast<float4*>(out + (size_t)pix * C + c) =
      make_float4(s.x / 6.0f, s.y / 6.0f, s.z / 6.0f, s.w / 6.0f);
}

void launch_avgpool32(const float* in, int N, int H, int W, int C, int in_ps, float* out, int Ho, int Wo,
                      hipStream_t s) {
  long total = (long)N * Ho * Wo * (C / 4);
  hipLaunchKernelGGL(avgpool32_kernel, dim3(blocks_for(total)), dim3(256), 0, s, in, N, H, W, C, in_ps, out, Ho, Wo);
}

// ----------------------------------------------------------------- FPN
// Residual squeeze-excitation output x + x*g (src/cpu/model.rs:1138-1142,
// :1188-1194), fused with the top-down nearest-upsample add
// (upsample_add_nchw, :1265-1320) or with the upsample-and-concat write
// (upsample_and_cat_nchw, :1322-1417): each input pixel is written as a
// rep x rep block into its channel slice of the concat tensor.
__global__ void gate_residual_kernel(const float* in, int N, int H, int W, int C, int in_ps, const float* gate,
                                     const float* upper, int up_ps, float* out, int out_ps, int rep) {
  const int C4 = C >> 2;
  long idx = (long)blockIdx.x * 256 + threadIdx.x;
  long total = (long)N * H * W * C4;
  if (idx >= total) return;
  int c = (int)(idx % C4) * 4;
  long pix = idx / C4;
  int x = (int)(pix % W);
  long t = pix / W;
  int y = (int)(t % H);
  int n = (int)(t / H);
  float4 v = *reinterpret_cast<const float4*>(in + (size_t)pix * in_ps + c);
  float4 g = *reinterpret_cast<const float4*>(gate + (size_t)n * C + c);
  v.x = residual_mul(v.x, g.x);
  v.y = residual_mul(v.y, g.y);
  v.z = residual_mul(v.z, g.z);
  v.w = residual_mul(v.w, g.w);
  if (upper) {
    int uh = H / 2, uw = W / 2;
    float4 u = *reinterpret_cast<const float4*>(upper + ((size_t)(n * uh + y / 2) * uw + x / 2) * up_ps + c);
    v.x = v.x + u.x;
    v.y = v.y + u.y;
    v.z = v.z + u.z;
    v.w = v.w + u.w;
  }
  if (rep == 1) {
    *reinterpret_cast<float4*>(out + (size_t)pix * out_ps + c) = v;
  } else {
    int OW = W * rep;
    for (int dy = 0; dy < rep; ++dy) {
      float* row = out + ((size_t)(n * H * rep + y * rep + dy) * OW + (size_t)x * rep) * out_ps + c;
      for (int dx = 0; dx < rep; ++dx) *reinterpret_cast<float4*>(row + (size_t)dx * out_ps) = v;
    }
  }
}

void launch_gate_residual(const float* in, int N, int H, int W, int C, int in_ps, const float* gate,
                          const float* upper, int up_ps, float* out, int out_ps, int rep, hipStream_t s) {
  long total = (long)N * H * W * (C / 4);
  hipLaunchKernelGGL(gate_residual_kernel, dim3(blocks_for(total)), dim3(256), 0, s, in, N, H, W, C, in_ps, gate,
                     upper, up_ps, out, out_ps, rep);
}

// ----------------------------------------------------------------- DB head
// Replaces WGSL `detector_head` / `deconv_phase` + `deconv_final`
// (src/gpu/shaders/detector_head.wgsl:52, deconv_phase.wgsl:105,
// deconv_final.wgsl:52).  Per input pixel at H/4 x W/4: conv_up (2x2 s2,
// BN folded, +bias, ReLU) then conv_final (2x2 s2 to one channel, +bias)
// and sigmoid (src/cpu/model.rs:1516-1520), 16 probabilities per lane.
// Weights: wu [c][o][4] (IOHW, folded), bu [o], wf [o][4].
template <int CH>
__global__ __launch_bounds__(256) void db_head_up_kernel(const float* in, int N, int H, int W, int in_ps,
                                                         const float* wu, const float* bu, const float* wf, float bf,
                                                         float* out) {
  __shared__ float s_wu[CH * CH * 4];
  __shared__ float s_bu[CH];
  __shared__ float s_wf[CH * 4];
  for (int i = threadIdx.x; i < CH * CH * 4; i += 256) s_wu[i] = wu[i];
  for (int i = threadIdx.x; i < CH; i += 256) s_bu[i] = bu[i];
  for (int i = threadIdx.x; i < CH * 4; i += 256) s_wf[i] = wf[i];
  __syncthreads();
  long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)N * H * W) return;
  int x = (int)(idx % W);
  long t = idx / W;
  int y = (int)(t % H);
  int n = (int)(t / H);
  float xin[CH];
  const float* src = in + (size_t)idx * in_ps;
#pragma unroll
  for (int c = 0; c < CH; c += 4) {
    float4 v = *reinterpret_cast<const float4*>(src + c);
    xin[c] = v.x;
    xin[c + 1] = v.y;
    xin[c + 2] = v.z;
    xin[c + 3] = v.w;
  }
  const int OW = 4 * W;
#pragma unroll
  for (int tap = 0; tap < 4; ++tap) {
    float f[4] = {0.f, 0.f, 0.f, 0.f};
    for (int o = 0; o < CH; ++o) {
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < CH; ++c) acc = fmaf(xin[c], s_wu[(c * CH + o) * 4 + tap], acc);
      float u = fmaxf(acc + s_bu[o], 0.0f);
#pragma unroll
      for (int q = 0; q < 4; ++q) f[q] = fmaf(u, s_wf[o * 4 + q], f[q]);
    }
    int yy = 4 * y + 2 * (tap >> 1);
    int xx = 4 * x + 2 * (tap & 1);
    float* o0 = out + ((size_t)n * 4 * H + yy) * OW + xx;
    float2 top = make_float2(1.0f / (1.0f + expf(-(f[0] + bf))), 1.0f / (1.0f + expf(-(f[1] + bf))));
    float2 bot = make_float2(1.0f / (1.0f + expf(-(f[2] + bf))), 1.0f / (1.0f + expf(-(f[3] + bf))));
    *reinterpret_cast<float2*>(o0) = top;
    *reinterpret_cast<float2*>(o0 + OW) = bot;
  }
}

void launch_db_head_up(const float* in, int N, int H, int W, int Ch, int in_ps, const float* wu, const float* bu,
                       const float* wf, float bf, float* out, hipStream_t s) {
  dim3 grid(blocks_for((long)N * H * W));
  switch (Ch) {
    case 16: hipLaunchKernelGGL(db_head_up_kernel<16>, grid, dim3(256), 0, s, in, N, H, W, in_ps, wu, bu, wf, bf, out); break;
    case 24: hipLaunchKernelGGL(db_head_up_kernel<24>, grid, dim3(256), 0, s, in, N, H, W, in_ps, wu, bu, wf, bf, out); break;
    case 64: hipLaunchKernelGGL(db_head_up_kernel<64>, grid, dim3(256), 0, s, in, N, H, W, in_ps, wu, bu, wf, bf, out); break;
    default: break;  // rejected by the planner
  }
}

// ----------------------------------------------------------------- LayerNorm
// Replaces WGSL `layer_norm` (src/gpu/shaders/layer_norm.wgsl:55); formula
// of layer_norm_in_place (src/cpu/kernels/mod.rs:2288-2313): two-pass mean
// and variance, out = (x - mean) * (inv_std * w) + b; one wave per row.
__global__ __launch_bounds__(256) void layer_norm_kernel(const float* in, int rows, int C, const float* w,
                                                         const float* b, float eps, const float* res, float* out) {
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* x = in + (size_t)row * C;
  float s = 0.0f;
  for (int c = lane; c < C; c += 64) s += x[c];
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  float mean = s / (float)C;
  float v = 0.0f;
  for (int c = lane; c < C; c += 64) {
    float d = x[c] - mean;
    v = fmaf(d, d, v);
  }
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  float var = v / (float)C;
  float inv = 1.0f / sqrtf(var + eps);
  float* y = out + (size_t)row * C;
  for (int c = lane; c < C; c += 64) {
    float r = fmaf(x[c] - mean, inv * w[c], b[c]);
    if (res) r = r + res[(size_t)row * C + c];
    y[c] = r;
  }
}

void launch_layer_norm(const float* in, int rows, int C, const float* w, const float* b, float eps, const float* res,
                       float* out, hipStream_t s) {
  hipLaunchKernelGGL(layer_norm_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0, s, in, rows, C, w, b, eps, res, out);
}

// ----------------------------------------------------------------- attention
// Replaces WGSL `attention_scores` + `attention_context`
// (src/gpu/shaders/attention.wgsl:62, :151); RecAttention::forward
// (src/cpu/model.rs:1703-1725): qkv laid out [B, T, 3, heads, hd];
// scores = (q . k) * hd^-0.5, max-subtracted softmax, context = P v.
// One block per (image, head, 16 query rows); the score rows stay in LDS.
constexpr int ATT_Q = 16;

__global__ __launch_bounds__(256) void attention_kernel(const float* qkv, int B, int T, int hidden, int heads,
                                                        float scale, float* out) {
  extern __shared__ float sc[];  // [ATT_Q][T]
  const int bh = blockIdx.x;
  const int b = bh / heads, h = bh - (bh / heads) * heads;
  const int t0 = blockIdx.y * ATT_Q;
  const int hd = hidden / heads;
  const int rows = min(ATT_Q, T - t0);
  const size_t stride = (size_t)3 * hidden;
  const float* base = qkv + (size_t)b * T * stride + h * hd;
  for (int i = threadIdx.x; i < rows * T; i += 256) {
    int r = i / T, u = i - (i / T) * T;
    const float* q = base + (size_t)(t0 + r) * stride;
    const float* k = base + (size_t)u * stride + hidden;
    float acc = 0.0f;
    for (int d = 0; d < hd; ++d) acc = fmaf(q[d], k[d], acc);
    sc[r * T + u] = __fmul_rn(acc, scale);
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int r = wave; r < rows; r += 4) {
    float* s = sc + r * T;
    float m = -INFINITY;
    for (int u = lane; u < T; u += 64) m = fmaxf(m, s[u]);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float sum = 0.0f;
    for (int u = lane; u < T; u += 64) {
      float e = expf(s[u] - m);
      s[u] = e;
      sum += e;
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    float rcp = 1.0f / sum;
    for (int u = lane; u < T; u += 64) s[u] *= rcp;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < rows * hd; i += 256) {
    int r = i / hd, d = i - (i / hd) * hd;
    const float* s = sc + r * T;
    const float* v = base + 2 * hidden + d;
    float acc = 0.0f;
    for (int u = 0; u < T; ++u) acc = fmaf(s[u], v[(size_t)u * stride], acc);
    out[((size_t)b * T + t0 + r) * hidden + h * hd + d] = acc;
  }
}

void launch_attention(const float* qkv, int B, int T, int hidden, int heads, float* out, hipStream_t s) {
  float scale = powf((float)(hidden / heads), -0.5f);
  dim3 grid(B * heads, (T + ATT_Q - 1) / ATT_Q);
  size_t lds = (size_t)ATT_Q * T * sizeof(float);
  hipLaunchKernelGGL(attention_kernel, grid, dim3(256), lds, s, qkv, B, T, hidden, heads, scale, out);
}

// ----------------------------------------------------------------- softmax
// Replaces WGSL `softmax` (src/gpu/shaders/softmax.wgsl:58); formula of
// softmax_in_place (src/cpu/kernels/mod.rs:2218-2245): max-subtracted exp,
// then multiplication by the reciprocal of the sum.  One block per row.
__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
  for (int o = 32; o > 0; o >>= 1) {
    float w = __shfl_xor(v, o);
    v = is_max ? fmaxf(v, w) : v + w;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
  return r;
}

__global__ __launch_bounds__(1024) void softmax_rows_kernel(float* x, int cols) {
  __shared__ float red[16];
  float* row = x + (size_t)blockIdx.x * cols;
  float m = -INFINITY;
  for (int i = threadIdx.x; i < cols; i += blockDim.x) m = fmaxf(m, row[i]);
  m = block_reduce(m, red, true);
  float s = 0.0f;
  for (int i = threadIdx.x; i < cols; i += blockDim.x) s += expf(row[i] - m);
  s = block_reduce(s, red, false);
  float rcp = 1.0f / s;
  for (int i = threadIdx.x; i < cols; i += blockDim.x) row[i] = expf(row[i] - m) * rcp;
}

void launch_softmax_rows(float* x, long rows, int cols, hipStream_t s) {
  hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)rows), dim3(1024), 0, s, x, cols);
}

// ----------------------------------------------------------------- preprocess
// The reference CPU preprocessing (src/preprocess/kernels.rs:94-170): quad
// bilinear source point, clamped; bilinear RGB rounded to an integer and
// clamped; v * (1/(255 std)) - mean/std as BGR; zero past content_width.
// Contraction is off so every product and sum rounds as in the reference.
__global__ void preprocess_kernel(PreParams p) {
#pragma clang fp contract(off)
  long idx = (long)blockIdx.x * 256 + threadIdx.x;
  long plane = (long)p.ch * p.cw;
  if (idx >= (long)p.N * plane) return;
  int n = (int)(idx / plane);
  long r = idx - n * plane;
  int y = (int)(r / p.cw);
  int x = (int)(r - (long)y * p.cw);
  int content = p.content_w[n];
  float b = 0.0f, g = 0.0f, rr = 0.0f;
  if (x < content) {
    const float* cr = p.corners + (size_t)n * 8;
    float v = ((float)y + 0.5f) / (float)p.ch;
    float omv = 1.0f - v;
    float u = ((float)x + 0.5f) / (float)content;
    float omu = 1.0f - u;
    float max_x = (float)(p.sw - 1), max_y = (float)(p.sh - 1);
    float sx = (cr[0] * omu + cr[2] * u) * omv + (cr[6] * omu + cr[4] * u) * v - 0.5f;
    float sy = (cr[1] * omu + cr[3] * u) * omv + (cr[7] * omu + cr[5] * u) * v - 0.5f;
    sx = fminf(fmaxf(sx, 0.0f), max_x);
    sy = fminf(fmaxf(sy, 0.0f), max_y);
    int x0 = (int)floorf(sx), y0 = (int)floorf(sy);
    int x1 = min(x0 + 1, p.sw - 1), y1 = min(y0 + 1, p.sh - 1);
    float tx = sx - (float)x0, ty = sy - (float)y0;
    const unsigned char* px = reinterpret_cast<const unsigned char*>(p.rgb);
    size_t o00 = ((size_t)y0 * p.sw + x0) * 3, o01 = ((size_t)y0 * p.sw + x1) * 3;
    size_t o10 = ((size_t)y1 * p.sw + x0) * 3, o11 = ((size_t)y1 * p.sw + x1) * 3;
    float rgb[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      float tl = px[o00 + c], tr = px[o01 + c], bl = px[o10 + c], br = px[o11 + c];
      float top = tl * (1.0f - tx) + tr * tx;
      float bot = bl * (1.0f - tx) + br * tx;
      rgb[c] = fminf(fmaxf(roundf(top * (1.0f - ty) + bot * ty), 0.0f), 255.0f);
    }
    b = rgb[2] * p.scale[0] + p.bias[0];
    g = rgb[1] * p.scale[1] + p.bias[1];
    rr = rgb[0] * p.scale[2] + p.bias[2];
  }
  if (p.nhwc) {
    *reinterpret_cast<float4*>(p.out + (size_t)idx * 4) = make_float4(b, g, rr, 0.0f);
  } else {
    float* o = p.out + (size_t)n * 3 * plane + r;
    o[0] = b;
    o[plane] = g;
    o[2 * plane] = rr;
  }
}

void launch_preprocess(const PreParams& p, hipStream_t s) {
  long total = (long)p.N * p.ch * p.cw;
  hipLaunchKernelGGL(preprocess_kernel, dim3(blocks_for(total)), dim3(256), 0, s, p);
}

}  // namespace ppocr
