// Fused pointwise pair of an LCNet block: y = W2 GELU(W1 x + b1) + b2, plus
// the block's residual.  Replaces two conv GEMM launches (and the HBM round
// trip of the 2C-channel hidden tensor) with one, as the reference CPU path
// fuses the pair per pixel tile (Conv2d::forward_pointwise_pair_gelu,
// src/cpu/backend.rs:443-695).
//
// A workgroup owns PB_M consecutive pixels.  Their input rows (C channels,
// multiplied by the SE gate when the block has one, rounded to fp32 as the
// unfused gather does; or, for blocks without SE, computed from the block
// input by its 3x3 depthwise token conv, the reference's depthwise ->
// pointwise strip fusion, src/cpu/backend.rs:697-816) are staged in LDS; the four waves compute the hidden
// tile GELU(x W1^T + b1) on the matrix cores (v_mfma_f32_16x16x4f32), 16
// hidden channels at a time, into a second LDS tile; then the output tile
// h W2^T + b2 (+ x for a residual block) from that, 16 output channels at a
// time.  Weights stream from L2.  The sums run in the order of the unfused
// kernel (K slices of 16 ascending, four MFMAs per slice), so results match
// it up to its split-K choices.  For one image the SE gate itself can be
// formed in the prologue from the token conv's partial channel sums (the
// squeeze-excitation's mean and two small convs, src/cpu/model.rs:456-493),
// so no separate gate launch precedes the pair.
#include "device_math.h"
#include "kernels.h"

namespace ppocr {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int PB_M = 32;  // pixels per workgroup (two 16-row MFMA tiles)

__device__ __forceinline__ void mfma4(f32x4& acc, float4 a, float4 b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, acc, 0, 0, 0);
}

// Two 16-row tiles of src (row stride lds floats, K columns) times 16 rows of
// w (row stride ldw, K columns): lane (lrow, g) reads k = k0 + 4g .. +3.
// The weight vectors come from L2 in chunks of KC slices, the next chunk's
// loads issued before the current chunk's products, so one load latency is
// exposed per column tile rather than one per K slice.
constexpr int KC = 4;

// Weight vectors at k >= kmax (k a multiple of 4) read as zero.
__device__ __forceinline__ float4 wvec(const float* p, int k, int kmax) {
  return k < kmax ? *reinterpret_cast<const float4*>(p) : make_float4(0.f, 0.f, 0.f, 0.f);
}

__device__ __forceinline__ void tile_product(const float* src, int lds, const float* wrow, int K, int lrow, int g,
                                             f32x4& acc0, f32x4& acc1, int kmax) {
  acc0 = f32x4{0.f, 0.f, 0.f, 0.f};
  acc1 = f32x4{0.f, 0.f, 0.f, 0.f};
  const float* a0p = src + lrow * lds + 4 * g;
  const float* a1p = src + (16 + lrow) * lds + 4 * g;
  const float* bp = wrow + 4 * g;
  const int nk = K / 16;
  float4 cur[KC];
#pragma unroll
  for (int i = 0; i < KC; ++i)
    if (i < nk) cur[i] = wvec(bp + i * 16, i * 16 + 4 * g, kmax);
  for (int c0 = 0; c0 < nk; c0 += KC) {
    float4 nxt[KC];
#pragma unroll
    for (int i = 0; i < KC; ++i)
      if (c0 + KC + i < nk) nxt[i] = wvec(bp + (c0 + KC + i) * 16, (c0 + KC + i) * 16 + 4 * g, kmax);
#pragma unroll
    for (int i = 0; i < KC; ++i) {
      if (c0 + i < nk) {
        const int k0 = (c0 + i) * 16;
        const float4 a0 = *reinterpret_cast<const float4*>(a0p + k0);
        const float4 a1 = *reinterpret_cast<const float4*>(a1p + k0);
        mfma4(acc0, a0, cur[i]);
        mfma4(acc1, a1, cur[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < KC; ++i) cur[i] = nxt[i];
  }
}

// DW: the input tile is the 3x3 depthwise conv of p.dw_in at the tile's
// pixels, summed as the depthwise kernels do (taps row-major, one fmaf per
// tap and channel, zeros for taps in the padding, then the bias).
template <bool GATE, bool RES, bool DW>
__global__ __launch_bounds__(256) void pointwise_pair_kernel(PairParams p) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int ldx = p.C + 4, ldh = p.H2 + 4;  // +4 floats: conflict-free 16-byte row reads
  float* xs = sm;                           // [PB_M][ldx]
  float* hs = sm + PB_M * ldx;              // [PB_M][ldh]
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lrow = lane & 15, g = lane >> 4;
  const int m0 = blockIdx.x * PB_M;

  // SE gate formed here (GATE with se_part, one image): gs[c] in the hidden
  // tile's LDS, free until the hidden products.  Lane (ph, q) sums partial
  // rows ph, ph + PH, ... of channel group q (eight loads in flight at a time),
  // the PH phase sums are added in order, then the two small convs run one
  // output per lane with their weights staged in LDS; every load is issued
  // before the first barrier.
  const float* gs = nullptr;
  if constexpr (GATE) {
    if (p.se_part) {
      float* g_lds = hs;             // [C]
      float* mean = hs + 64;         // [C]
      float* hid = hs + 128;         // [Cr]
      float* w1s = hs + 144;         // [Cr][C]
      float* w2s = w1s + p.se_Cr * p.C;  // [C][Cr]
      float4* red = reinterpret_cast<float4*>(xs);  // [PH][C / 4], free until the input tile
      const int C4 = p.C >> 2, PH = 256 / C4;
      const int nw1 = p.se_Cr * p.C / 4, nw2 = p.C * p.se_Cr / 4;  // float4 of W1, W2 (<= 256 each)
      // (Loads under if, not ?:, which the compiler turns into a load from
      // either the buffer or a zero on the stack.)
      float4 w1v = make_float4(0.f, 0.f, 0.f, 0.f), w2v = w1v;
      if (tid < nw1) w1v = reinterpret_cast<const float4*>(p.se_w1)[tid];
      if (tid < nw2) w2v = reinterpret_cast<const float4*>(p.se_w2)[tid];
      float b1v = 0.0f, b2v = 0.0f;
      if (tid < p.se_Cr) b1v = p.se_b1[tid];
      if (tid < p.C) b2v = p.se_b2[tid];
      const int q = tid % C4, ph = tid / C4;
      float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int r0 = 0; r0 < p.se_P; r0 += 8 * PH) {  // eight rows per lane in flight at a time
        float4 v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int row = r0 + ph + k * PH;
          v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (ph < PH && row < p.se_P)
            v[k] = *reinterpret_cast<const float4*>(p.se_part + (size_t)row * p.C + 4 * q);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k)
          sum = make_float4(sum.x + v[k].x, sum.y + v[k].y, sum.z + v[k].z, sum.w + v[k].w);
      }
      if (ph < PH) red[ph * C4 + q] = sum;
      if (tid < nw1) reinterpret_cast<float4*>(w1s)[tid] = w1v;
      if (tid < nw2) reinterpret_cast<float4*>(w2s)[tid] = w2v;
      __syncthreads();
      if (tid < C4) {
        float4 t = red[tid];
        for (int k = 1; k < PH; ++k) {
          const float4 r = red[k * C4 + tid];
          t = make_float4(t.x + r.x, t.y + r.y, t.z + r.z, t.w + r.w);
        }
        const float count = (float)p.HW;
        mean[4 * tid + 0] = t.x / count;
        mean[4 * tid + 1] = t.y / count;
        mean[4 * tid + 2] = t.z / count;
        mean[4 * tid + 3] = t.w / count;
      }
      __syncthreads();
      if (tid < p.se_Cr) {
        float a = 0.0f;
        for (int c = 0; c < p.C; ++c) a = fmaf(w1s[tid * p.C + c], mean[c], a);
        hid[tid] = fmaxf(a + b1v, 0.0f);
      }
      __syncthreads();
      if (tid < p.C) {
        float a = 0.0f;
        for (int j = 0; j < p.se_Cr; ++j) a = fmaf(w2s[tid * p.se_Cr + j], hid[j], a);
        g_lds[tid] = act_apply(p.se_act, a + b2v);
      }
      __syncthreads();
      gs = g_lds;
    }
  }

  // Input tile, gated; rows past M are zero.
  const int c4 = p.C >> 2;
  for (int i = tid; i < PB_M * c4; i += 256) {
    const int r = i / c4, c = (i - r * c4) * 4;
    const int m = m0 + r;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (DW && m < p.M) {
      const int n = m / p.HW, rem = m - n * p.HW;
      const int oy = rem / p.dw_wo, ox = rem - oy * p.dw_wo;
      const float* img = p.dw_in + (size_t)n * p.dw_h * p.dw_w * p.dw_ps + c;
#pragma unroll
      for (int ky = 0; ky < 3; ++ky) {
        const int iy = oy * p.dw_sh - p.dw_pt + ky;
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) {
          const int ix = ox * p.dw_sw - p.dw_pl + kx;
          const float4 x = (unsigned)iy < (unsigned)p.dw_h && (unsigned)ix < (unsigned)p.dw_w
                               ? *reinterpret_cast<const float4*>(img + ((size_t)iy * p.dw_w + ix) * p.dw_ps)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
          const float4 w = *reinterpret_cast<const float4*>(p.dw_wt + (size_t)(ky * 3 + kx) * p.C + c);
          v.x = fmaf(x.x, w.x, v.x);
          v.y = fmaf(x.y, w.y, v.y);
          v.z = fmaf(x.z, w.z, v.z);
          v.w = fmaf(x.w, w.w, v.w);
        }
      }
      if (p.dw_b) {
        const float4 b = *reinterpret_cast<const float4*>(p.dw_b + c);
        v = make_float4(v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w);
      }
    } else if (m < p.M) {
      v = *reinterpret_cast<const float4*>(p.in + (size_t)m * p.in_ps + c);
      if constexpr (GATE) {
        const float4 gt = gs ? *reinterpret_cast<const float4*>(gs + c)
                             : *reinterpret_cast<const float4*>(p.gate + (size_t)(m / p.HW) * p.C + c);
        v = make_float4(__fmul_rn(v.x, gt.x), __fmul_rn(v.y, gt.y), __fmul_rn(v.z, gt.z), __fmul_rn(v.w, gt.w));
      }
    }
    *reinterpret_cast<float4*>(xs + r * ldx + c) = v;
  }
  __syncthreads();

  // Hidden tile: lane (lrow, g) of column tile ct holds rows 4g + v (and
  // 16 + 4g + v) of hidden channel ct * 16 + lrow.
  for (int ct = wave; ct < p.H2 / 16; ct += 4) {
    f32x4 acc0, acc1;
    const int col = ct * 16 + lrow;
    tile_product(xs, ldx, p.w1 + (size_t)col * p.ldw1, p.C, lrow, g, acc0, acc1, p.C);
    const float b = p.b1 ? p.b1[col] : 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      hs[(4 * g + v) * ldh + col] = act_apply(ACT_GELU, acc0[v] + b);
      hs[(16 + 4 * g + v) * ldh + col] = act_apply(ACT_GELU, acc1[v] + b);
    }
  }
  __syncthreads();

  // Output tile.
  for (int ct = wave; ct < p.Co / 16; ct += 4) {
    f32x4 acc0, acc1;
    const int col = ct * 16 + lrow;
    tile_product(hs, ldh, p.w2 + (size_t)col * p.ldw2, p.H2, lrow, g, acc0, acc1, p.H2);
    const float b = p.b2 ? p.b2[col] : 0.0f;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const f32x4& acc = half ? acc1 : acc0;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = half * 16 + 4 * g + v;
        const int m = m0 + row;
        if (m >= p.M) continue;
        float o = acc[v] + b;
        if constexpr (RES) o = o + xs[row * ldx + col];  // the gated input, as the unfused residual
        p.out[(size_t)m * p.out_ps + col] = o;
      }
    }
  }
}

// LayerNorm fused into the linear layer that reads it (RecBlock's
// layer_norm1 -> qkv and layer_norm2 -> fc1, src/cpu/model.rs:1768-1772):
// out = act(LN(x) W^T + b).  A workgroup owns 32 rows and 64 output
// columns (grid y), one 16-column tile per wave.  Eight lanes normalise one
// row: each holds up to LN_V float4 of it in registers, the row's sum and
// squared deviations are reduced over the eight lanes, and the normalised
// values fma(x - mean, inv * w, b) (layer_norm_in_place's formula) go to LDS,
// zero-padded to a multiple of 16 features; each column group redoes this
// for its rows (32 x K reads against 64 x K weights).  The product then runs
// as in the pair kernel (columns past N computed on row N - 1 of W and not
// stored).
constexpr int LN_V = 8;  // float4 per lane: K <= 8 lanes * 8 * 4 = 256

__global__ __launch_bounds__(256) void ln_linear_kernel(LnLinearParams p) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int K16 = (p.K + 15) & ~15;
  const int ldx = K16 + 4;
  float* xs = sm;  // [PB_M][ldx]
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lrow = lane & 15, g = lane >> 4;
  const int m0 = blockIdx.x * PB_M;
  {
    const int r = tid >> 3, sub = tid & 7;  // row r of the tile, lane sub of its eight
    const int m = m0 + r;
    const int k4 = p.K >> 2;
    float4 v[LN_V];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < LN_V; ++i) {
      const int j = sub + 8 * i;
      v[i] = m < p.M && j < k4 ? *reinterpret_cast<const float4*>(p.in + (size_t)m * p.in_ps + 4 * j)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
      s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
    for (int o = 1; o < 8; o <<= 1) s += __shfl_xor(s, o);
    const float mean = s / (float)p.K;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < LN_V; ++i) {
      if (sub + 8 * i < k4) {
        const float a = v[i].x - mean, b = v[i].y - mean, c = v[i].z - mean, d = v[i].w - mean;
        q = fmaf(a, a, q);
        q = fmaf(b, b, q);
        q = fmaf(c, c, q);
        q = fmaf(d, d, q);
      }
    }
    for (int o = 1; o < 8; o <<= 1) q += __shfl_xor(q, o);
    const float inv = 1.0f / sqrtf(q / (float)p.K + p.eps);
    float* y = xs + r * ldx;
#pragma unroll
    for (int i = 0; i < LN_V; ++i) {
      const int j = sub + 8 * i;
      if (4 * j >= K16) continue;
      float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
      if (m < p.M && j < k4) {
        const float4 w = *reinterpret_cast<const float4*>(p.ln_w + 4 * j);
        const float4 b = *reinterpret_cast<const float4*>(p.ln_b + 4 * j);
        o = make_float4(fmaf(v[i].x - mean, inv * w.x, b.x), fmaf(v[i].y - mean, inv * w.y, b.y),
                        fmaf(v[i].z - mean, inv * w.z, b.z), fmaf(v[i].w - mean, inv * w.w, b.w));
      }
      *reinterpret_cast<float4*>(y + 4 * j) = o;
    }
  }
  __syncthreads();
  {
    const int ct = blockIdx.y * 4 + wave;
    if (ct * 16 >= p.N) return;  // after the only barrier
    f32x4 acc0, acc1;
    const int col = ct * 16 + lrow;
    const int wr = col < p.N ? col : p.N - 1;
    tile_product(xs, ldx, p.w + (size_t)wr * p.ldw, K16, lrow, g, acc0, acc1, p.K);
    if (col >= p.N) return;
    const float b = p.b ? p.b[col] : 0.0f;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const f32x4& acc = half ? acc1 : acc0;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + half * 16 + 4 * g + v;
        if (m < p.M) p.out[(size_t)m * p.out_ps + col] = act_apply(p.act, acc[v] + b);
      }
    }
  }
}

}  // namespace

size_t ln_linear_lds(int K) { return (size_t)PB_M * (((K + 15) & ~15) + 4) * sizeof(float); }

bool ln_linear_supported(int K, int N, int dt) {
  return dt == DT_F32 && K % 4 == 0 && K <= 32 * LN_V && N >= 1;
}

void launch_ln_linear(const LnLinearParams& p, hipStream_t s) {
  const dim3 grid((unsigned)((p.M + PB_M - 1) / PB_M), (unsigned)((p.N + 63) / 64));
  hipLaunchKernelGGL(ln_linear_kernel, grid, dim3(256), ln_linear_lds(p.K), s, p);
}

bool pointwise_pair_supported(int C, int H2, int Co, int dt) {
  return dt == DT_F32 && C % 16 == 0 && H2 % 16 == 0 && Co % 16 == 0 && pointwise_pair_lds(C, H2) <= (160u << 10);
}

bool pair_se_fold_supported(int N, int C, int H2, int Cr, int P) {
  // The phase sums fit the input tile's LDS (C >= 32), the staged weights,
  // means and gate the hidden tile's, and a lane sums at most 32 rows.
  return N == 1 && C >= 32 && C <= 64 && C % 4 == 0 && Cr >= 1 && Cr <= 16 && (C * Cr) % 4 == 0 && P >= 1 &&
         P <= 32 * (256 / (C / 4)) && 144 + 2 * C * Cr <= PB_M * (H2 + 4);
}

size_t pointwise_pair_lds(int C, int H2) { return (size_t)PB_M * ((C + 4) + (H2 + 4)) * sizeof(float); }

void launch_pointwise_pair(const PairParams& p, hipStream_t s) {
  const dim3 grid((unsigned)((p.M + PB_M - 1) / PB_M));
  const size_t lds = pointwise_pair_lds(p.C, p.H2);
  const bool gate = p.gate != nullptr || p.se_part != nullptr, res = p.residual != 0;
  if (p.dw_in) {
    if (res)
      hipLaunchKernelGGL((pointwise_pair_kernel<false, true, true>), grid, dim3(256), lds, s, p);
    else
      hipLaunchKernelGGL((pointwise_pair_kernel<false, false, true>), grid, dim3(256), lds, s, p);
  } else if (gate && res)
    hipLaunchKernelGGL((pointwise_pair_kernel<true, true, false>), grid, dim3(256), lds, s, p);
  else if (gate)
    hipLaunchKernelGGL((pointwise_pair_kernel<true, false, false>), grid, dim3(256), lds, s, p);
  else if (res)
    hipLaunchKernelGGL((pointwise_pair_kernel<false, true, false>), grid, dim3(256), lds, s, p);
  else
    hipLaunchKernelGGL((pointwise_pair_kernel<false, false, false>), grid, dim3(256), lds, s, p);
}

}  // namespace ppocr
