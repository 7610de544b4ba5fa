// Bandwidth-bound kernels of the detector and recognizer: depthwise conv,
// squeeze-excitation, FPN gate/upsample/concat, pools, the fused DB head
// tail, LayerNorm, attention, row softmax and image preprocessing.
//
// All activations are NHWC with C % 4 == 0, so one lane moves four channels
// (16 B as fp32, 8 B as bf16) and consecutive lanes touch consecutive
// segments: every global access of these kernels is coalesced.  Arithmetic
// is fp32 for both storage types.
#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <type_traits>

#include "device_math.h"

namespace ppocr {

static inline unsigned blocks_for(long n, int per = 256) { return (unsigned)((n + per - 1) / per); }

#define DISPATCH_DT(dt, ...)            \
  do {                                  \
    if ((dt) == DT_BF16) {              \
      using T = bf16;                   \
      __VA_ARGS__;                      \
    } else {                            \
      using T = float;                  \
      __VA_ARGS__;                      \
    }                                   \
  } while (0)

__device__ __forceinline__ float4 f4_act(int act, float4 v) {
  return make_float4(act_apply(act, v.x), act_apply(act, v.y), act_apply(act, v.z), act_apply(act, v.w));
}

__device__ __forceinline__ float4 f4_sum(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// ----------------------------------------------------------------- depthwise
// Replaces WGSL `depthwise` (src/gpu/shaders/depthwise.wgsl:77); semantics of
// the reference CPU depthwise (src/cpu/ops.rs:385-826): zero padding, bias,
// activation, then optional residual add (x + act(dw(x) + b)).  This generic
// form serves the shapes the strip and tiled kernels below do not cover.
template <typename T>
__global__ __launch_bounds__(256) void depthwise_kernel(DwParams p) {
  const T* in = static_cast<const T*>(p.in);
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
    const T* row = in + (size_t)(n * p.H + iy) * p.W * p.in_ps + c;
    const float* wrow = p.wt + (size_t)ky * p.kw * p.C + c;
    for (int kx = 0; kx < p.kw; ++kx) {
      int ix = ox * p.sw - p.pl + kx;
      if (ix < 0 || ix >= p.W) continue;
      float4 x = ld4<T>(row + (size_t)ix * p.in_ps);
      float4 w = *reinterpret_cast<const float4*>(wrow + (size_t)kx * p.C);
      acc.x = fmaf(x.x, w.x, acc.x);
      acc.y = fmaf(x.y, w.y, acc.y);
      acc.z = fmaf(x.z, w.z, acc.z);
      acc.w = fmaf(x.w, w.w, acc.w);
    }
  }
  if (p.bias) acc = f4_sum(acc, *reinterpret_cast<const float4*>(p.bias + c));
  acc = f4_act(p.act, acc);
  if (p.res) acc = f4_sum(ld4<T>(static_cast<const T*>(p.res) + (size_t)pix * p.res_ps + c), acc);
  st4<T>(static_cast<T*>(p.out) + (size_t)pix * p.out_ps + c, acc);
}

// LDS-tiled stride-1 depthwise.  A block computes a TY x TX output tile of
// 4 * C4B channels (C4B lanes per pixel).  The input tile with its halo and
// the taps are staged once in LDS as fp32; each lane then slides a register
// window of XR + KW - 1 pixels along x to produce XR outputs, so every
// staged value is reused KW x KH times from registers/LDS instead of being
// re-read from the caches.  Per tap row a lane reads XR + KW - 1 window and
// KW tap vectors for KW * XR * 4 FMAs.  The 7x7 and 9x9 layers take 16-row
// tiles of 16 channels (less halo per output row; measured faster than
// wider XR, which costs occupancy).  Taps accumulate in (ky, kx) order as
// the generic kernel does.
// SH, SW: the layer's strides (the input tile spans (TY - 1) SH + KH rows
// and (TX - 1) SW + KW columns; the gate-residual prologue is stride 1).
template <typename T, int KH, int KW, int TY, int XR = 4, int C4B = 8, int SH = 1, int SW = 1>
__global__ __launch_bounds__(256) void depthwise_tiled_kernel(DwParams p) {
  constexpr int XG = 256 / (C4B * TY);    // lane groups along x
  constexpr int TX = XG * XR;
  constexpr int IH = (TY - 1) * SH + KH, IW = (TX - 1) * SW + KW;
  constexpr int WN = (XR - 1) * SW + KW;  // input pixels of a lane's window row
  static_assert(KH != 7 || (SH == 1 && SW == 1), "the gate-residual prologue is stride 1");
  constexpr int IWP = IW | 1;  // odd row pitch (pixels)
  __shared__ float4 tile[IH * IWP * C4B];
  __shared__ float4 taps[KH * KW * C4B];
  const T* in = static_cast<const T*>(p.in);

  // Tiles numbered channel block fastest, then x, y, image; XCD-contiguous
  // ranges as in depthwise_wave_kernel.
  const int cblocks = (p.C + 4 * C4B - 1) / (4 * C4B);
  const int tiles_x = (p.Wo + TX - 1) / TX, tiles_y = (p.Ho + TY - 1) / TY;
  const int total = tiles_x * tiles_y * cblocks * p.N;
  const int t = (blockIdx.x & 7) * ((total + 7) / 8) + (blockIdx.x >> 3);
  if (t >= total) return;  // grid padding, before any barrier
  const int txy = t / cblocks;
  const int n = txy / (tiles_x * tiles_y);
  const int blk = txy - n * tiles_x * tiles_y;  // tile within the image
  const int ch0 = (t - txy * cblocks) * 4 * C4B;
  const int oy0 = blk / tiles_x * TY, ox0 = blk % tiles_x * TX;
  const int tid = threadIdx.x;

  // Tap vector of this lane (one per lane at most), loaded with the tile so
  // that both wait on one memory latency.
  static_assert(KH * KW * C4B <= 256, "one tap vector per lane");
  float4 tap = f4_zero();
  if (tid < KH * KW * C4B) {
    const int c = ch0 + (tid % C4B) * 4;
    if (c < p.C) tap = *reinterpret_cast<const float4*>(p.wt + (size_t)(tid / C4B) * p.C + c);
  }

  {
    // A lane keeps one channel group (256 is a multiple of C4B) and steps
    // through the tile's pixels; the image base and channel test are hoisted.
    static_assert(256 % C4B == 0, "fixed channel group per lane");
    const int c4 = tid % C4B;
    const int c = ch0 + c4 * 4;
    const bool cok = c < p.C;
    const T* base = in + (size_t)n * p.H * p.W * p.in_ps + c;
    constexpr int STEP = 256 / C4B, NL = (IH * IW + STEP - 1) / STEP;
    // Gate-residual prologue, as in depthwise_wave_kernel (7x7 layers only:
    // the 3x3 instances keep their registers for occupancy).
    if (KH == 7 && p.gr_gate) {
      const float4 gt = cok ? *reinterpret_cast<const float4*>(p.gr_gate + (size_t)n * p.C + c) : f4_zero();
      const int uh = p.H / 2, uw = p.W / 2;
      const T* up = p.gr_up ? static_cast<const T*>(p.gr_up) + (size_t)n * uh * uw * p.gr_up_ps + c : nullptr;
      // All of this lane's loads (the conv output, then the upper level's)
      // are issued before the first store.
      float4 hv[NL], uv[NL];
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const int px = tid / C4B + i * STEP;
        const int iy = px / IW, ix = px - iy * IW;
        const int gy = oy0 - p.pt + iy, gx = ox0 - p.pl + ix;
        const bool ok = px < IH * IW && cok && (unsigned)gy < (unsigned)p.H && (unsigned)gx < (unsigned)p.W;
        hv[i] = ok ? ld4<T>(base + ((size_t)gy * p.W + gx) * p.in_ps) : f4_zero();
        uv[i] = ok && up ? ld4<T>(up + ((size_t)(gy / 2) * uw + gx / 2) * p.gr_up_ps) : f4_zero();
      }
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const int px = tid / C4B + i * STEP;
        if (px >= IH * IW) break;
        const int iy = px / IW, ix = px - iy * IW;
        const int gy = oy0 - p.pt + iy, gx = ox0 - p.pl + ix;
        float4 x = f4_zero();
        if (cok && (unsigned)gy < (unsigned)p.H && (unsigned)gx < (unsigned)p.W) {
          const float4 h = hv[i];
          x = make_float4(residual_mul(h.x, gt.x), residual_mul(h.y, gt.y), residual_mul(h.z, gt.z),
                          residual_mul(h.w, gt.w));
          if (up) x = f4_sum(x, uv[i]);
          x = round4<T>(x);
          if (p.gr_out && (unsigned)(iy - p.pt) < (unsigned)TY && (unsigned)(ix - p.pl) < (unsigned)TX)
            st4<T>(static_cast<T*>(p.gr_out) + ((size_t)(n * p.H + gy) * p.W + gx) * p.gr_out_ps + c, x);
        }
        tile[(iy * IWP + ix) * C4B + c4] = x;
      }
    } else {
    // All of this lane's loads are issued before the first LDS store.
    float4 v[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int px = tid / C4B + i * STEP;
      const int iy = px / IW, ix = px - iy * IW;
      const int gy = oy0 * SH - p.pt + iy, gx = ox0 * SW - p.pl + ix;
      v[i] = f4_zero();
      if (px < IH * IW && cok && (unsigned)gy < (unsigned)p.H && (unsigned)gx < (unsigned)p.W)
        v[i] = ld4<T>(base + ((size_t)gy * p.W + gx) * p.in_ps);
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int px = tid / C4B + i * STEP;
      const int iy = px / IW, ix = px - iy * IW;
      if (px < IH * IW) tile[(iy * IWP + ix) * C4B + c4] = v[i];
    }
    }
  }
  if (tid < KH * KW * C4B) taps[tid] = tap;
  __syncthreads();

  // Channel groups fastest, then rows, then x groups: with C4B * TY = 64 a
  // wave reads one x group, and the odd row pitch puts its lanes on
  // consecutive 16-byte bank slots (4 cycles per ds_read_b128; x groups
  // inside a wave measured 8).
  const int c4 = tid % C4B;
  const int ty = (tid / C4B) % TY;
  const int xg = tid / (C4B * TY);
  float4 acc[XR];
#pragma unroll
  for (int r = 0; r < XR; ++r) acc[r] = f4_zero();
  // One row window live at a time keeps the kernel free of register spills.
#pragma unroll 1
  for (int ky = 0; ky < KH; ++ky) {
    float4 win[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) win[j] = tile[((ty * SH + ky) * IWP + xg * XR * SW + j) * C4B + c4];
#pragma unroll
    for (int kx = 0; kx < KW; ++kx) {
      float4 w = taps[(ky * KW + kx) * C4B + c4];
#pragma unroll
      for (int r = 0; r < XR; ++r) {
        acc[r].x = fmaf(win[r * SW + kx].x, w.x, acc[r].x);
        acc[r].y = fmaf(win[r * SW + kx].y, w.y, acc[r].y);
        acc[r].z = fmaf(win[r * SW + kx].z, w.z, acc[r].z);
        acc[r].w = fmaf(win[r * SW + kx].w, w.w, acc[r].w);
      }
    }
  }
  const int c = ch0 + c4 * 4;
  const int oy = oy0 + ty;
  const bool cin = c < p.C;
  float4 b = p.bias && cin ? *reinterpret_cast<const float4*>(p.bias + c) : f4_zero();
  float4 sum = f4_zero();  // this lane's stored outputs, for the SE partial sums
#pragma unroll
  for (int r = 0; r < XR; ++r) {
    int ox = ox0 + xg * XR + r;
    if (!cin || oy >= p.Ho || ox >= p.Wo) break;
    float4 v = acc[r];
    if (p.bias) v = f4_sum(v, b);
    v = f4_act(p.act, v);
    size_t pix = (size_t)(n * p.Ho + oy) * p.Wo + ox;
    if (p.res) v = f4_sum(ld4<T>(static_cast<const T*>(p.res) + pix * p.res_ps + c), v);
    T* o = static_cast<T*>(p.out) + pix * p.out_ps + c;
    st4<T>(o, v);
    if (p.se_part) sum = f4_sum(sum, round4<T>(v));
  }
  if (p.se_part) {
    // Channel sums of the block's outputs (in the storage type, as a later
    // reader sees them): lanes of one channel group add in a fixed order.
    __syncthreads();  // every lane is done with the input tile
    tile[tid] = sum;
    __syncthreads();
    if (tid < C4B && ch0 + tid * 4 < p.C) {
      float4 sums = tile[tid];
      for (int k = 1; k < 256 / C4B; ++k) sums = f4_sum(sums, tile[k * C4B + tid]);
      *reinterpret_cast<float4*>(p.se_part + ((size_t)n * tiles_x * tiles_y + blk) * p.C + ch0 + tid * 4) = sums;
    }
  }
}

// The bf16 form of depthwise_tiled_kernel for channel counts in groups of 8
// with 16-byte-aligned pixels: a lane owns 8 channels (16-byte loads and
// stores, half the lanes and workgroups per pixel of the 4-channel form),
// the input tile is staged in LDS as packed bf16 and unpacked as a lane
// reads its window.  The 4-channel form ran as long as the fp32 kernel on
// the same maps (its cost is per lane and workgroup, not per byte); this one
// measured 1.31-1.37x on the recognizer's 6- and 12-row maps and 1.28x on
// the detector's 104 x 184 map, with bit-identical outputs (same taps in the
// same (ky, kx) order).  SE partial sums as the 4-channel form leaves them.
// SH, SW: the layer's strides (the input tile spans (TY - 1) SH + KH rows
// and (TX - 1) SW + KW columns).
template <int KH, int KW, int TY, int XR, int C8B, int SH = 1, int SW = 1>
__global__ __launch_bounds__(256) void depthwise_tiled8_kernel(DwParams p) {
  constexpr int XG = 256 / (C8B * TY);  // lane groups along x
  constexpr int TX = XG * XR;
  constexpr int IH = (TY - 1) * SH + KH, IW = (TX - 1) * SW + KW;
  constexpr int WN = (XR - 1) * SW + KW;  // input pixels of a lane's window row
  constexpr int IWP = IW | 1;  // odd row pitch (pixels)
  static_assert(IH * IWP * C8B >= 512, "the SE reduction reuses the tile");
  __shared__ uint4 tile[IH * IWP * C8B];
  constexpr int NT = KH * KW * C8B * 2;  // tap float4s of the block
  constexpr int TIT = (NT + 255) / 256;
  __shared__ float4 taps[NT];
  const bf16* in = static_cast<const bf16*>(p.in);

  const int cblocks = (p.C + 8 * C8B - 1) / (8 * C8B);
  const int tiles_x = (p.Wo + TX - 1) / TX, tiles_y = (p.Ho + TY - 1) / TY;
  const int total = tiles_x * tiles_y * cblocks * p.N;
  const int t = (blockIdx.x & 7) * ((total + 7) / 8) + (blockIdx.x >> 3);
  if (t >= total) return;  // grid padding, before any barrier
  const int txy = t / cblocks;
  const int n = txy / (tiles_x * tiles_y);
  const int blk = txy - n * tiles_x * tiles_y;  // tile within the image
  const int ch0 = (t - txy * cblocks) * 8 * C8B;
  const int oy0 = blk / tiles_x * TY, ox0 = blk % tiles_x * TX;
  const int tid = threadIdx.x;

  // The block's taps, loaded with the tile.
  float4 tv[TIT];
#pragma unroll
  for (int it = 0; it < TIT; ++it) {
    const int i = tid + 256 * it;
    const int c = ch0 + (i % (2 * C8B)) * 4;
    tv[it] = i < NT && c < p.C ? *reinterpret_cast<const float4*>(p.wt + (size_t)(i / (2 * C8B)) * p.C + c) : f4_zero();
  }
  {
    static_assert(256 % C8B == 0, "fixed channel group per lane");
    const int c8 = tid % C8B;
    const int c = ch0 + c8 * 8;
    const bool cok = c < p.C;
    const bf16* base = in + (size_t)n * p.H * p.W * p.in_ps + c;
    constexpr int STEP = 256 / C8B, NL = (IH * IW + STEP - 1) / STEP;
    uint4 v[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int px = tid / C8B + i * STEP;
      const int iy = px / IW, ix = px - iy * IW;
      const int gy = oy0 * SH - p.pt + iy, gx = ox0 * SW - p.pl + ix;
      v[i] = make_uint4(0, 0, 0, 0);
      if (px < IH * IW && cok && (unsigned)gy < (unsigned)p.H && (unsigned)gx < (unsigned)p.W)
        v[i] = *reinterpret_cast<const uint4*>(base + ((size_t)gy * p.W + gx) * p.in_ps);
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int px = tid / C8B + i * STEP;
      const int iy = px / IW, ix = px - iy * IW;
      if (px < IH * IW) tile[(iy * IWP + ix) * C8B + c8] = v[i];
    }
  }
#pragma unroll
  for (int it = 0; it < TIT; ++it)
    if (tid + 256 * it < NT) taps[tid + 256 * it] = tv[it];
  __syncthreads();

  // Channel groups fastest, then rows, then x groups (as the 4-channel form).
  const int c8 = tid % C8B;
  const int ty = (tid / C8B) % TY;
  const int xg = tid / (C8B * TY);
  float4 acc[XR][2];
#pragma unroll
  for (int r = 0; r < XR; ++r) acc[r][0] = acc[r][1] = f4_zero();
#pragma unroll 1
  for (int ky = 0; ky < KH; ++ky) {
    float4 win[WN][2];
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const uint4 u = tile[((ty * SH + ky) * IWP + xg * XR * SW + j) * C8B + c8];
      win[j][0] = unpack_bf16x4(u.x, u.y);
      win[j][1] = unpack_bf16x4(u.z, u.w);
    }
#pragma unroll
    for (int kx = 0; kx < KW; ++kx) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float4 w = taps[((ky * KW + kx) * C8B + c8) * 2 + h];
#pragma unroll
        for (int r = 0; r < XR; ++r) {
          acc[r][h].x = fmaf(win[r * SW + kx][h].x, w.x, acc[r][h].x);
          acc[r][h].y = fmaf(win[r * SW + kx][h].y, w.y, acc[r][h].y);
          acc[r][h].z = fmaf(win[r * SW + kx][h].z, w.z, acc[r][h].z);
          acc[r][h].w = fmaf(win[r * SW + kx][h].w, w.w, acc[r][h].w);
        }
      }
    }
  }
  const int c = ch0 + c8 * 8;
  const int oy = oy0 + ty;
  const bool cin = c < p.C;
  float4 b0 = f4_zero(), b1 = f4_zero();
  if (p.bias && cin) {
    b0 = *reinterpret_cast<const float4*>(p.bias + c);
    b1 = *reinterpret_cast<const float4*>(p.bias + c + 4);
  }
  float4 sum0 = f4_zero(), sum1 = f4_zero();  // this lane's stored outputs, for the SE partial sums
#pragma unroll
  for (int r = 0; r < XR; ++r) {
    const int ox = ox0 + xg * XR + r;
    if (!cin || oy >= p.Ho || ox >= p.Wo) break;
    float4 v0 = acc[r][0], v1 = acc[r][1];
    if (p.bias) {
      v0 = f4_sum(v0, b0);
      v1 = f4_sum(v1, b1);
    }
    v0 = f4_act(p.act, v0);
    v1 = f4_act(p.act, v1);
    const size_t pix = (size_t)(n * p.Ho + oy) * p.Wo + ox;
    if (p.res) {
      const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const bf16*>(p.res) + pix * p.res_ps + c);
      v0 = f4_sum(unpack_bf16x4(u.x, u.y), v0);
      v1 = f4_sum(unpack_bf16x4(u.z, u.w), v1);
    }
    const uint4 o = make_uint4(pack_bf16x2(v0.x, v0.y), pack_bf16x2(v0.z, v0.w), pack_bf16x2(v1.x, v1.y),
                               pack_bf16x2(v1.z, v1.w));
    *reinterpret_cast<uint4*>(static_cast<bf16*>(p.out) + pix * p.out_ps + c) = o;
    if (p.se_part) {
      sum0 = f4_sum(sum0, unpack_bf16x4(o.x, o.y));
      sum1 = f4_sum(sum1, unpack_bf16x4(o.z, o.w));
    }
  }
  if (p.se_part) {
    // Channel sums of the block's outputs as stored; lanes of one channel
    // group add in a fixed order.
    __syncthreads();  // every lane is done with the input tile
    float4* red = reinterpret_cast<float4*>(tile);
    red[2 * tid] = sum0;
    red[2 * tid + 1] = sum1;
    __syncthreads();
    if (tid < 2 * C8B && ch0 + tid * 4 < p.C) {
      // tid = 2 * (channel group) + half
      float4 sums = red[tid];
      for (int k = 1; k < 256 / C8B; ++k) sums = f4_sum(sums, red[k * 2 * C8B + tid]);
      *reinterpret_cast<float4*>(p.se_part + ((size_t)n * tiles_x * tiles_y + blk) * p.C + ch0 + tid * 4) = sums;
    }
  }
}

// LDS-tiled stride-1 depthwise for large kernels with wave-uniform taps: a
// block computes a 16 x 16 output tile of 16 channels and each wave one
// group of 4 channels, so all lanes of a wave read the same tap vector (an
// LDS broadcast: the block's taps are staged in LDS with the tile; read from
// memory per tap row they cost the 9x9 layers 1.1x, the 5x5 even, although
// staging them takes the 9x9 from four workgroups per CU to three).
// Lane (ty, xg) = (lane / 4, lane % 4) slides a window of 4 + KW - 1 pixels
// of tile row ty + ky for 4 outputs; a tap row costs 4 + KW - 1 LDS reads for
// 4 * KW * 4 FMAs.  The input tile is stored per channel group with an odd
// row pitch (IWP float4).  (This lane order measured 2.2 LDS conflict cycles
// per instruction against 5.4 with rows fastest, at equal speed.)  The
// results go back through LDS (pixel-major, channel groups fastest, padded
// pitches) so the stores, bias / activation / residual included, run with
// four lanes per 64-byte pixel.  Taps accumulate in (ky, kx) order as in the
// generic kernel.  Tiles are numbered channel block fastest, then x, y,
// image, and workgroup b takes tile (b % 8) * per + b / 8 (per = tiles / 8
// rounded up): the hardware deals workgroups to the 8 XCDs in turn, so each
// XCD walks a contiguous tile range and the two 64-byte halves of a
// 128-byte line (adjacent channel blocks) meet in one L2 (1.05-1.17x on the
// neck's maps).
constexpr int kDwWaveT = 16, kDwWaveG = 4;

template <typename T, int KH, int KW>
__global__ __launch_bounds__(256) void depthwise_wave_kernel(DwParams p) {
  constexpr int TY = kDwWaveT, TX = kDwWaveT, G = kDwWaveG;  // G channel groups of 4 per block
  constexpr int IH = TY + KH - 1, IW = TX + KW - 1;
  constexpr int IWP = IW | 1;                  // odd pitch
  constexpr int OPX = 5, OROW = TX * OPX + 1;  // staged output pitch (float4)
  static_assert(G * IH * IWP >= TY * OROW, "output staging fits the tile");
  constexpr int NT = KH * KW * G, TIT = (NT + 255) / 256;  // tap vectors of the block
  __shared__ float4 tile[G * IH * IWP];
  __shared__ float4 taps[NT];
  const T* in = static_cast<const T*>(p.in);

  const int cblocks = (p.C + 4 * G - 1) / (4 * G);
  const int tiles_x = (p.Wo + TX - 1) / TX, tiles_y = (p.Ho + TY - 1) / TY;
  const int total = tiles_x * tiles_y * cblocks * p.N;
  const int t = (blockIdx.x & 7) * ((total + 7) / 8) + (blockIdx.x >> 3);
  if (t >= total) return;  // grid padding, before any barrier
  const int cb = t % cblocks;
  const int txy = t / cblocks;
  const int n = txy / (tiles_x * tiles_y);
  const int ch0 = cb * 4 * G;
  const int oy0 = (txy / tiles_x) % tiles_y * TY, ox0 = txy % tiles_x * TX;
  const int tid = threadIdx.x;

  // The block's taps go to LDS with the tile (loaded with it).
  float4 tv[TIT];
#pragma unroll
  for (int it = 0; it < TIT; ++it) {
    const int i = tid + 256 * it;
    const int c = ch0 + (i % G) * 4;
    tv[it] = i < NT && c < p.C ? *reinterpret_cast<const float4*>(p.wt + (size_t)(i / G) * p.C + c) : f4_zero();
  }
  {
    // A lane keeps one channel group and steps through the tile's pixels 64
    // at a time; the image base and channel test are hoisted, and the loads
    // of all its pixels are issued before the first LDS write.
    constexpr int NPX = IH * IW, PPI = 256 / G, IT = (NPX + PPI - 1) / PPI;
    const int g = tid & (G - 1);
    const int c = ch0 + g * 4;
    const bool cok = c < p.C;
    const T* base = in + (size_t)n * p.H * p.W * p.in_ps + c;
    float4 v[IT];
    if (p.gr_gate) {
      // x = in + in * gate (+ up2(upper)), rounded as gate_residual_kernel
      // stores it; pixels of the tile's output block also go to gr_out.
      const float4 gt = cok ? *reinterpret_cast<const float4*>(p.gr_gate + (size_t)n * p.C + c) : f4_zero();
      const int uh = p.H / 2, uw = p.W / 2;
      const T* up = p.gr_up ? static_cast<const T*>(p.gr_up) + (size_t)n * uh * uw * p.gr_up_ps + c : nullptr;
      float4 u[IT];
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int px = tid / G + PPI * it;
        const int iy = px / IW, ix = px - iy * IW;
        const int gy = oy0 - p.pt + iy, gx = ox0 - p.pl + ix;
        v[it] = u[it] = f4_zero();
        if (px < NPX && cok && (unsigned)gy < (unsigned)p.H && (unsigned)gx < (unsigned)p.W) {
          v[it] = ld4<T>(base + ((size_t)gy * p.W + gx) * p.in_ps);
          if (up) u[it] = ld4<T>(up + ((size_t)(gy / 2) * uw + gx / 2) * p.gr_up_ps);
        }
      }
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int px = tid / G + PPI * it;
        if (px >= NPX) break;
        const int iy = px / IW, ix = px - iy * IW;
        const int gy = oy0 - p.pt + iy, gx = ox0 - p.pl + ix;
        float4 x = f4_zero();
        if (cok && (unsigned)gy < (unsigned)p.H && (unsigned)gx < (unsigned)p.W) {
          const float4 h = v[it];
          x = make_float4(residual_mul(h.x, gt.x), residual_mul(h.y, gt.y), residual_mul(h.z, gt.z),
                          residual_mul(h.w, gt.w));
          if (up) x = f4_sum(x, u[it]);
          x = round4<T>(x);
          if (p.gr_out && (unsigned)(iy - p.pt) < (unsigned)TY && (unsigned)(ix - p.pl) < (unsigned)TX)
            st4<T>(static_cast<T*>(p.gr_out) + ((size_t)(n * p.H + gy) * p.W + gx) * p.gr_out_ps + c, x);
        }
        tile[(g * IH + iy) * IWP + ix] = x;
      }
    } else {
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int px = tid / G + PPI * it;
        const int iy = px / IW, ix = px - iy * IW;
        const int gy = oy0 - p.pt + iy, gx = ox0 - p.pl + ix;
        v[it] = f4_zero();
        if (px < NPX && cok && (unsigned)gy < (unsigned)p.H && (unsigned)gx < (unsigned)p.W)
          v[it] = ld4<T>(base + ((size_t)gy * p.W + gx) * p.in_ps);
      }
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int px = tid / G + PPI * it;
        if (px >= NPX) break;
        const int iy = px / IW, ix = px - iy * IW;
        tile[(g * IH + iy) * IWP + ix] = v[it];
      }
    }
  }
#pragma unroll
  for (int it = 0; it < TIT; ++it)
    if (tid + 256 * it < NT) taps[tid + 256 * it] = tv[it];
  __syncthreads();

  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // this wave's channel group
  const int lane = tid & 63;
  const int ty = lane >> 2, xg = lane & 3;
  const int c = ch0 + wave * 4;
  const bool cin = c < p.C;
  float4 acc[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) acc[r] = f4_zero();
  const float4* trow = tile + (wave * IH + ty) * IWP + xg * 4;
  // Three tap rows per iteration (5x5 layers 1.04x with the taps read from
  // memory, registers unchanged).
#pragma unroll 3
  for (int ky = 0; ky < KH; ++ky) {
    float4 w[KW];
#pragma unroll
    for (int kx = 0; kx < KW; ++kx) w[kx] = taps[(ky * KW + kx) * G + wave];
    float4 win[4 + KW - 1];
#pragma unroll
    for (int j = 0; j < 4 + KW - 1; ++j) win[j] = trow[ky * IWP + j];
#pragma unroll
    for (int kx = 0; kx < KW; ++kx) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[r].x = fmaf(win[r + kx].x, w[kx].x, acc[r].x);
        acc[r].y = fmaf(win[r + kx].y, w[kx].y, acc[r].y);
        acc[r].z = fmaf(win[r + kx].z, w[kx].z, acc[r].z);
        acc[r].w = fmaf(win[r + kx].w, w[kx].w, acc[r].w);
      }
    }
  }
  const float4 b = p.bias && cin ? *reinterpret_cast<const float4*>(p.bias + c) : f4_zero();
  __syncthreads();  // every wave is done with the input tile
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float4 v = acc[r];
    if (p.bias) v = f4_sum(v, b);
    tile[ty * OROW + (xg * 4 + r) * OPX + wave] = f4_act(p.act, v);
  }
  __syncthreads();
  for (int i = tid; i < TY * TX * G; i += 256) {
    const int g = i % G;
    const int px = i / G;
    const int ox = ox0 + px % TX, oy = oy0 + px / TX;
    const int cc = ch0 + g * 4;
    if (cc >= p.C || ox >= p.Wo || oy >= p.Ho) continue;
    float4 v = tile[(px / TX) * OROW + (px % TX) * OPX + g];
    const size_t pix = (size_t)(n * p.Ho + oy) * p.Wo + ox;
    if (p.res) v = f4_sum(ld4<T>(static_cast<const T*>(p.res) + pix * p.res_ps + cc), v);
    st4<T>(static_cast<T*>(p.out) + pix * p.out_ps + cc, v);
  }
}

// bf16 depthwise k x k (k = 5, 7, 9, stride 1) on the matrix cores.  For one
// channel and tap row ky, a 16 x 16 output tile is a 16x16x32 product
//   out[y][x] += sum_k in[y + ky][x0 + k] * T_ky[k][x],  T_ky[k][x] = w[ky][k - x]
// (T_ky is zero outside 0 <= k - x < kw): A rows are input rows read straight
// from LDS, B is the Toeplitz matrix of the tap row, packed on the host
// (depthwise_mfma_table), and 16 + kw - 1 <= 32 input columns cover the tile.
// Products of bf16 values are exact and accumulate in fp32, in K order per
// tap row instead of the VALU kernels' (ky, kx) order.
// A workgroup takes a 32 x 32 output tile of 8 channels (16 bytes a pixel,
// one load or store per lane; 8-byte accesses measured 1.4 TB/s on the
// neck's largest map): wave w owns channels 2w and 2w + 1, each as four
// 16 x 16 MFMA tiles.  The input tile sits in LDS channel-major,
// [8][rows][28 dwords]: a 112-byte row pitch puts the 16 rows an A-fragment
// read touches on distinct banks, and the columns past the tile's input
// (read as the zero-weight tail of the last K group) are written as zeros.
// Outputs are staged in the same LDS as four planes of channel pairs.
// Registers are held to four waves per SIMD, what the LDS allows (the tile
// loads issued ahead would otherwise cost a wave: three measured slower).
constexpr int kDwMfmaT = 32, kDwMfmaP = 28, kDwMfmaC = 8;  // tile side, LDS row pitch (dwords), channels
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

template <int K>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void depthwise_mfma_kernel(DwParams p) {
  constexpr int T = kDwMfmaT, P = kDwMfmaP, CB = kDwMfmaC;
  constexpr int IH = T + K - 1, IW = T + K - 1;
  static_assert(16 + K - 1 <= 32 && IW <= 2 * (P - 4), "a tile's K window fits the padded row");
  // Staged outputs: one plane of channel pairs per wave, [row][col] float2
  // with a row pitch of 72 floats, so the 32 lanes of a float2 write phase
  // (16 columns of rows r and r + 4) cover the 64 banks once.
  constexpr int SP = 2 * T + 8, PLANE = T * SP;
  constexpr int TILE = CB * IH * P, STAGE = 4 * PLANE;
  __shared__ __align__(16) uint32_t lds[TILE > STAGE ? TILE : STAGE];

  const int cgroups = p.C / CB;
  const int tiles_x = (p.Wo + T - 1) / T, tiles_y = (p.Ho + T - 1) / T;
  const int total = tiles_x * tiles_y * cgroups * p.N;
  const int t = (blockIdx.x & 7) * ((total + 7) / 8) + (blockIdx.x >> 3);
  if (t >= total) return;  // grid padding, before any barrier
  const int txy = t / cgroups;
  const int ch0 = (t - txy * cgroups) * CB;
  const int n = txy / (tiles_x * tiles_y);
  const int oy0 = (txy / tiles_x) % tiles_y * T, ox0 = txy % tiles_x * T;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;

  // This wave's B fragments (per channel, one per tap row), issued before
  // the tile loads.
  bf16x8_t bw[2][K];
  {
    const uint4* tab = static_cast<const uint4*>(p.wtab) + (size_t)(ch0 + 2 * wave) * K * 64 + lane;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int ky = 0; ky < K; ++ky) bw[c][ky] = __builtin_bit_cast(bf16x8_t, tab[(c * K + ky) * 64]);
  }

  // Input tile: pixel pairs along x, transposed to 8 channel planes.  A
  // lane issues the loads of all its pixel pairs before its first LDS write.
  {
    const uint4* in = static_cast<const uint4*>(p.in);  // 8 bf16 channels per pixel
    constexpr int NQ = IH * (P - 4), IT = (NQ + 255) / 256;
    uint4 u0[IT], u1[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int q = tid + 256 * it;
      const int row = q / (P - 4), xp = q - row * (P - 4);
      const int gy = oy0 - p.pt + row, gx = ox0 - p.pl + 2 * xp;
      u0[it] = u1[it] = make_uint4(0, 0, 0, 0);
      if (q < NQ && (unsigned)gy < (unsigned)p.H) {
        const size_t rowpix = (size_t)(n * p.H + gy) * p.W;
        if (2 * xp < IW && (unsigned)gx < (unsigned)p.W) u0[it] = in[((rowpix + gx) * p.in_ps + ch0) / CB];
        if (2 * xp + 1 < IW && (unsigned)(gx + 1) < (unsigned)p.W)
          u1[it] = in[((rowpix + gx + 1) * p.in_ps + ch0) / CB];
      }
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int q = tid + 256 * it;
      if (q >= NQ) break;
      const int row = q / (P - 4), xp = q - row * (P - 4);
      uint32_t* dst = lds + row * P + xp;
      const uint32_t a[4] = {u0[it].x, u0[it].y, u0[it].z, u0[it].w}, b[4] = {u1[it].x, u1[it].y, u1[it].z, u1[it].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dst[(2 * j) * IH * P] = (a[j] & 0xFFFFu) | (b[j] << 16);
        dst[(2 * j + 1) * IH * P] = (a[j] >> 16) | (b[j] & 0xFFFF0000u);
      }
    }
  }
  __syncthreads();

  floatx4_t acc[2][2][2];  // [channel][ty][tx]
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[c][i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    // Lane (row lane % 16, K group lane / 16) reads 8 columns of an input row.
    const uint32_t* base = lds + ((2 * wave + c) * IH + (lane & 15)) * P + (lane >> 4) * 4;
#pragma unroll
    for (int ky = 0; ky < K; ++ky)
#pragma unroll
      for (int ty = 0; ty < 2; ++ty)
#pragma unroll
        for (int tx = 0; tx < 2; ++tx) {
          const uint4 a = *reinterpret_cast<const uint4*>(base + (16 * ty + ky) * P + 8 * tx);
          acc[c][ty][tx] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), bw[c][ky],
                                                                    acc[c][ty][tx], 0, 0, 0);
        }
  }
  __syncthreads();  // every wave is done with the input tile

  // acc[c][ty][tx][r] is output (16 ty + 4 (lane / 16) + r, 16 tx + lane % 16)
  // of channel 2 wave + c; the wave's two channels go out as one float2.
  float* stage = reinterpret_cast<float*>(lds);
  {
    float* plane = stage + wave * PLANE;
#pragma unroll
    for (int ty = 0; ty < 2; ++ty)
#pragma unroll
      for (int tx = 0; tx < 2; ++tx)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          *reinterpret_cast<float2*>(plane + (16 * ty + 4 * (lane >> 4) + r) * SP + 2 * (16 * tx + (lane & 15))) =
              make_float2(acc[0][ty][tx][r], acc[1][ty][tx][r]);
  }
  __syncthreads();
  float4 b0 = f4_zero(), b1 = f4_zero();
  if (p.bias) {
    b0 = *reinterpret_cast<const float4*>(p.bias + ch0);
    b1 = *reinterpret_cast<const float4*>(p.bias + ch0 + 4);
  }
#pragma unroll
  for (int k = 0; k < T * T / 256; ++k) {
    const int px = tid + 256 * k;
    const int row = px / T, col = px % T;
    const int oy = oy0 + row, ox = ox0 + col;
    if (oy >= p.Ho || ox >= p.Wo) continue;
    const float* sp = stage + row * SP + 2 * col;
    const float2 c01 = *reinterpret_cast<const float2*>(sp), c23 = *reinterpret_cast<const float2*>(sp + PLANE);
    const float2 c45 = *reinterpret_cast<const float2*>(sp + 2 * PLANE);
    const float2 c67 = *reinterpret_cast<const float2*>(sp + 3 * PLANE);
    float4 v0 = make_float4(c01.x, c01.y, c23.x, c23.y);
    float4 v1 = make_float4(c45.x, c45.y, c67.x, c67.y);
    if (p.bias) v0 = f4_sum(v0, b0), v1 = f4_sum(v1, b1);
    v0 = f4_act(p.act, v0);
    v1 = f4_act(p.act, v1);
    const size_t pix = (size_t)(n * p.Ho + oy) * p.Wo + ox;
    if (p.res) {
      const bf16* rp = static_cast<const bf16*>(p.res) + pix * p.res_ps + ch0;
      v0 = f4_sum(ld4<bf16>(rp), v0);
      v1 = f4_sum(ld4<bf16>(rp + 4), v1);
    }
    uint4 o;
    o.x = pack_bf16x2(v0.x, v0.y);
    o.y = pack_bf16x2(v0.z, v0.w);
    o.z = pack_bf16x2(v1.x, v1.y);
    o.w = pack_bf16x2(v1.z, v1.w);
    *reinterpret_cast<uint4*>(static_cast<bf16*>(p.out) + pix * p.out_ps + ch0) = o;
  }
}

template <int K>
static void launch_dw_mfma(const DwParams& p, hipStream_t s) {
  const long tiles =
      (long)((p.Wo + kDwMfmaT - 1) / kDwMfmaT) * ((p.Ho + kDwMfmaT - 1) / kDwMfmaT) * p.N * (p.C / kDwMfmaC);
  hipLaunchKernelGGL((depthwise_mfma_kernel<K>), dim3((unsigned)((tiles + 7) / 8 * 8)), dim3(256), 0, s, p);
}

bool depthwise_uses_mfma(int kh, int kw, int sh, int sw, int dt, int Ho, int C) {
  return dt == DT_BF16 && kh == kw && (kh == 5 || kh == 7 || kh == 9) && sh == 1 && sw == 1 && Ho >= 16 &&
         C % kDwMfmaC == 0;
}

size_t depthwise_mfma_table_size(int c, int k) { return (size_t)c * k * 64 * 8; }

void depthwise_mfma_table(const float* w, int c, int k, uint16_t* out) {
  for (int ch = 0; ch < c; ++ch)
    for (int ky = 0; ky < k; ++ky)
      for (int lane = 0; lane < 64; ++lane)
        for (int i = 0; i < 8; ++i) {
          const int j = 8 * (lane / 16) + i - lane % 16;
          const float v = j >= 0 && j < k ? w[((size_t)ch * k + ky) * k + j] : 0.f;
          uint32_t u;
          memcpy(&u, &v, 4);
          out[(((size_t)ch * k + ky) * 64 + lane) * 8 + i] =
              (u & 0x7FFFFFFFu) > 0x7F800000u ? (uint16_t)((u >> 16) | 0x40u)
                                               : (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
        }
}

// Depthwise as vertical strips, no LDS: a lane owns four channels of R
// consecutive output rows at one x (vertical stride SH, horizontal stride
// p.sw).  It walks the (R - 1) * SH + KH input rows of its strip once,
// loading the KW pixels of each row (the neighbouring x lanes load the same
// pixels, so they come from L1/L2 and HBM sees each input about once), and
// adds each row into every output row it touches.  The taps stay in
// registers.  Output row r receives its input rows in increasing ky and
// each row in increasing kx: the (ky, kx) tap order of the generic kernel.
// Lanes run channels fastest, then x, so every load and store of a wave is
// one contiguous run.
template <typename T, int KH, int KW, int R, int SH>
__global__ __launch_bounds__(256) void depthwise_strip_kernel(DwParams p) {
  const T* in = static_cast<const T*>(p.in);
  const int C4 = p.C >> 2;
  const int strips = (p.Ho + R - 1) / R;
  long idx = (long)blockIdx.x * 256 + threadIdx.x;
  const long total = (long)p.N * strips * p.Wo * C4;
  if (idx >= total) return;
  const int c4 = (int)(idx % C4);
  long t = idx / C4;
  const int ox = (int)(t % p.Wo);
  t /= p.Wo;
  const int strip = (int)(t % strips);
  const int n = (int)(t / strips);
  const int c = c4 * 4;
  const int oy0 = strip * R;
  const int rows = min(R, p.Ho - oy0);

  float4 w[KH * KW];
#pragma unroll
  for (int i = 0; i < KH * KW; ++i) w[i] = *reinterpret_cast<const float4*>(p.wt + (size_t)i * p.C + c);
  float4 acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = f4_zero();

  const T* img = in + (size_t)n * p.H * p.W * p.in_ps + c;
  const int ix0 = ox * p.sw - p.pl;
#pragma unroll
  for (int j = 0; j < (R - 1) * SH + KH; ++j) {  // input row oy0 * SH - pt + j
    const int iy = oy0 * SH - p.pt + j;
    if (iy < 0 || iy >= p.H) continue;
    float4 x[KW];
#pragma unroll
    for (int kx = 0; kx < KW; ++kx) {
      const int ix = ix0 + kx;
      x[kx] = ix >= 0 && ix < p.W ? ld4<T>(img + ((size_t)iy * p.W + ix) * p.in_ps) : f4_zero();
    }
    // Output row r = (j - ky) / SH takes this row as its tap row ky.
#pragma unroll
    for (int ky = KH - 1; ky >= 0; --ky) {
      if (j < ky || (j - ky) % SH != 0) continue;
      const int r = (j - ky) / SH;
      if (r >= R) continue;
#pragma unroll
      for (int kx = 0; kx < KW; ++kx) {
        const float4 wk = w[ky * KW + kx];
        acc[r].x = fmaf(x[kx].x, wk.x, acc[r].x);
        acc[r].y = fmaf(x[kx].y, wk.y, acc[r].y);
        acc[r].z = fmaf(x[kx].z, wk.z, acc[r].z);
        acc[r].w = fmaf(x[kx].w, wk.w, acc[r].w);
      }
    }
  }
  const float4 b = p.bias ? *reinterpret_cast<const float4*>(p.bias + c) : f4_zero();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r >= rows) break;
    float4 v = acc[r];
    if (p.bias) v = f4_sum(v, b);
    v = f4_act(p.act, v);
    const size_t pix = (size_t)(n * p.Ho + oy0 + r) * p.Wo + ox;
    if (p.res) v = f4_sum(ld4<T>(static_cast<const T*>(p.res) + pix * p.res_ps + c), v);
    st4<T>(static_cast<T*>(p.out) + pix * p.out_ps + c, v);
  }
}

template <typename T, int KH, int KW, int R, int SH>
static void launch_dw_strip(const DwParams& p, hipStream_t s) {
  const long total = (long)p.N * ((p.Ho + R - 1) / R) * p.Wo * (p.C / 4);
  hipLaunchKernelGGL((depthwise_strip_kernel<T, KH, KW, R, SH>), dim3(blocks_for(total)), dim3(256), 0, s, p);
}

template <typename T, int KH, int KW, int TY, int XR = 4, int C4B = 8, int SH = 1, int SW = 1>
static void launch_dw_tiled(const DwParams& p, hipStream_t s) {
  constexpr int TX = 256 / (C4B * TY) * XR;
  const long tiles = (long)((p.Wo + TX - 1) / TX) * ((p.Ho + TY - 1) / TY) * p.N * ((p.C + 4 * C4B - 1) / (4 * C4B));
  hipLaunchKernelGGL((depthwise_tiled_kernel<T, KH, KW, TY, XR, C4B, SH, SW>), dim3((unsigned)((tiles + 7) / 8 * 8)),
                     dim3(256), 0, s, p);
}

template <typename T, int KH, int KW>
static void launch_dw_wave(const DwParams& p, hipStream_t s) {
  // One workgroup per tile, the count rounded up to a multiple of the XCDs.
  const long tiles = (long)((p.Wo + kDwWaveT - 1) / kDwWaveT) * ((p.Ho + kDwWaveT - 1) / kDwWaveT) * p.N *
                     ((p.C + 4 * kDwWaveG - 1) / (4 * kDwWaveG));
  hipLaunchKernelGGL((depthwise_wave_kernel<T, KH, KW>), dim3((unsigned)((tiles + 7) / 8 * 8)), dim3(256), 0, s, p);
}

// The launch shape of the tiled 3x3 kernels, the ones that can leave SE
// partial sums (stride 1 and more than 4 output rows): 8 lanes per pixel
// (32 fp32 or 64 bf16 channels), 2 outputs per lane along x (1.03-1.22x
// over 4 outputs on the detector's fp32 maps, more blocks for the same
// work and less tail; on bf16 maps 1.03-1.04x on the recognizer's 6- and
// 12-row maps too), 8-row tiles except for bf16 maps whose height is a
// multiple of 4 but not of 8, which take 4-row tiles, and bf16 maps of 6
// rows, which take 2-row tiles, so that no lane row is idle (the
// recognizer's 12-row maps 1.23-1.25x, its 6-row maps 1.07x, the
// detector's 52-row map 1.03x; measured on the isolated layers, identical
// outputs).
// bf16 maps of 3 and 4 rows (the recognizer's last stage) take the tiled
// kernel with 4-row tiles too, in place of the vertical strips (1.38x on
// 256x3x80x768, identical outputs), and leave SE sums.
constexpr int kDw3C4B = 8, kDw3XR = 2;
constexpr int dw3_ty(int dt, int ho) {
  return dt != DT_BF16                   ? 8
         : ho <= 4                       ? 4
         : ho % 8 != 0 && ho % 4 == 0    ? 4
         : ho % 4 != 0 && ho % 2 == 0 && ho <= 8 ? 2
                                         : 8;
}
static int dw3_tx(int dt, int ho) { return 256 / (kDw3C4B * dw3_ty(dt, ho)) * kDw3XR; }
// Stride-1 3x3 layers on the tiled kernels: more than 4 output rows, or 3
// or 4 rows in bf16.
static bool dw3_tiled_rows(int dt, int ho) { return ho > 4 || (dt == DT_BF16 && ho >= 3); }

int depthwise_se_blocks(const DwParams& p) {
  if (!(p.kh == 3 && p.kw == 3 && p.sh == 1 && p.sw == 1 && dw3_tiled_rows(p.dt, p.Ho))) return 0;
  const int tx = dw3_tx(p.dt, p.Ho), ty = dw3_ty(p.dt, p.Ho);
  return ((p.Wo + tx - 1) / tx) * ((p.Ho + ty - 1) / ty);
}

// bf16 3x3 stride-1 layers take the 8-channel tiled kernel when every pixel
// access is a whole 16-byte group.
static bool dw3_tiled8(const DwParams& p) {
  return p.dt == DT_BF16 && p.C % 8 == 0 && p.in_ps % 8 == 0 && p.out_ps % 8 == 0 && (!p.res || p.res_ps % 8 == 0) &&
         (((uintptr_t)p.in | (uintptr_t)p.out | (uintptr_t)p.res) & 15) == 0;
}

template <int KH, int KW, int TY, int XR, int C8B, int SH = 1, int SW = 1>
static void launch_dw_tiled8(const DwParams& p, hipStream_t s) {
  constexpr int TX = 256 / (C8B * TY) * XR;
  const long tiles = (long)((p.Wo + TX - 1) / TX) * ((p.Ho + TY - 1) / TY) * p.N * ((p.C + 8 * C8B - 1) / (8 * C8B));
  hipLaunchKernelGGL((depthwise_tiled8_kernel<KH, KW, TY, XR, C8B, SH, SW>), dim3((unsigned)((tiles + 7) / 8 * 8)),
                     dim3(256), 0, s, p);
}

template <typename T>
static void launch_dw_typed(const DwParams& p, hipStream_t s) {
  if (p.gr_gate) {  // the gate-residual prologue: wave (5x5, 9x9) and tiled (7x7) kernels
    if (p.kh == 5 && p.kw == 5 && p.sh == 1 && p.sw == 1) return launch_dw_wave<T, 5, 5>(p, s);
    if (p.kh == 7 && p.kw == 7 && p.sh == 1 && p.sw == 1) return launch_dw_tiled<T, 7, 7, 16, 4, 4>(p, s);
    if (p.kh == 9 && p.kw == 9 && p.sh == 1 && p.sw == 1) return launch_dw_wave<T, 9, 9>(p, s);
    return;  // depthwise_gate_residual_supported() rules this out at plan time
  }
  if constexpr (sizeof(T) == 2) {
    // 16-byte pixel accesses: strides and base addresses in whole 8-channel groups.
    const bool aligned = p.in_ps % kDwMfmaC == 0 && p.out_ps % kDwMfmaC == 0 &&
                         (!p.res || p.res_ps % kDwMfmaC == 0) &&
                         (((uintptr_t)p.in | (uintptr_t)p.out | (uintptr_t)p.res) & 15) == 0;
    if (p.wtab && !p.se_part && aligned && depthwise_uses_mfma(p.kh, p.kw, p.sh, p.sw, DT_BF16, p.Ho, p.C)) {
      if (p.kh == 5) return launch_dw_mfma<5>(p, s);
      if (p.kh == 7) return launch_dw_mfma<7>(p, s);
      return launch_dw_mfma<9>(p, s);
    }
  }
  // 3x3 with vertical stride 2 (stage entries), and maps of at most 4 rows
  // (the recognizer's last stage), where the LDS tile would load its halo
  // rows for only a few output rows: vertical strips.
  if (p.kh == 3 && p.kw == 3 && p.sh == 2) {
    // Stage entries on the tiled kernels: stride (2, 1) (the recognizer's)
    // with the bf16 stride-1 tile rows of the output height, stride (2, 2)
    // (the detector's) with 4-row tiles of one output per lane (over the
    // strips, identical outputs: bf16 on the 8-channel kernel 1.66-1.85x
    // and 1.38-1.72x, fp32 1.06-1.12x and 1.10-1.37x).
    if (p.sw == 2) {
      if constexpr (sizeof(T) == 2)
        if (dw3_tiled8(p)) return launch_dw_tiled8<3, 3, 4, 1, kDw3C4B, 2, 2>(p, s);
      return launch_dw_tiled<T, 3, 3, 4, 1, kDw3C4B, 2, 2>(p, s);
    }
    if (p.sw == 1) {
      const int ty = dw3_ty(DT_BF16, p.Ho);
      if constexpr (sizeof(T) == 2)
        if (dw3_tiled8(p))
          return ty == 2   ? launch_dw_tiled8<3, 3, 2, kDw3XR, kDw3C4B, 2, 1>(p, s)
                 : ty == 4 ? launch_dw_tiled8<3, 3, 4, kDw3XR, kDw3C4B, 2, 1>(p, s)
                           : launch_dw_tiled8<3, 3, 8, kDw3XR, kDw3C4B, 2, 1>(p, s);
      return ty == 2   ? launch_dw_tiled<T, 3, 3, 2, kDw3XR, kDw3C4B, 2, 1>(p, s)
             : ty == 4 ? launch_dw_tiled<T, 3, 3, 4, kDw3XR, kDw3C4B, 2, 1>(p, s)
                       : launch_dw_tiled<T, 3, 3, 8, kDw3XR, kDw3C4B, 2, 1>(p, s);
    }
    return launch_dw_strip<T, 3, 3, 3, 2>(p, s);
  }
  if (p.kh == 3 && p.kw == 3 && p.sh == 1 && !dw3_tiled_rows(p.dt, p.Ho))
    return p.Ho == 3 ? launch_dw_strip<T, 3, 3, 3, 1>(p, s) : launch_dw_strip<T, 3, 3, 4, 1>(p, s);
  if (p.sh == 1 && p.sw == 1) {
    if (p.kh == 3 && p.kw == 3) {
      if constexpr (sizeof(T) == 2) {
        const int ty = dw3_ty(DT_BF16, p.Ho);
        if (dw3_tiled8(p))
          return ty == 2   ? launch_dw_tiled8<3, 3, 2, kDw3XR, kDw3C4B>(p, s)
                 : ty == 4 ? launch_dw_tiled8<3, 3, 4, kDw3XR, kDw3C4B>(p, s)
                           : launch_dw_tiled8<3, 3, 8, kDw3XR, kDw3C4B>(p, s);
        return ty == 2   ? launch_dw_tiled<T, 3, 3, 2, kDw3XR, kDw3C4B>(p, s)
               : ty == 4 ? launch_dw_tiled<T, 3, 3, 4, kDw3XR, kDw3C4B>(p, s)
                         : launch_dw_tiled<T, 3, 3, 8, kDw3XR, kDw3C4B>(p, s);
      }
      return launch_dw_tiled<T, 3, 3, 8, kDw3XR, kDw3C4B>(p, s);
    }
    // 5x5 and 9x9: wave-uniform taps (1.1-1.2x the tiled kernel's per-lane taps);
    // 7x7 (32 channels here) measured even: 16-row tiles of 16 channels.
    if (p.kh == 5 && p.kw == 5) return launch_dw_wave<T, 5, 5>(p, s);
    if (p.kh == 7 && p.kw == 7) return launch_dw_tiled<T, 7, 7, 16, 4, 4>(p, s);
    if (p.kh == 9 && p.kw == 9) return launch_dw_wave<T, 9, 9>(p, s);
    if (p.kh == 1 && p.kw == 5 && p.Ho == 1) return launch_dw_tiled<T, 1, 5, 1>(p, s);
    if (p.kh == 1 && p.kw == 7 && p.Ho == 1) return launch_dw_tiled<T, 1, 7, 1>(p, s);
  }
  long total = (long)p.N * p.Ho * p.Wo * (p.C / 4);
  hipLaunchKernelGGL(depthwise_kernel<T>, dim3(blocks_for(total)), dim3(256), 0, s, p);
}

void launch_depthwise(const DwParams& p, hipStream_t s) { DISPATCH_DT(p.dt, launch_dw_typed<T>(p, s)); }

bool depthwise_gate_residual_supported(int kh, int kw, int sh, int sw) {
  return kh == kw && (kh == 5 || kh == 7 || kh == 9) && sh == 1 && sw == 1;
}

const char* depthwise_kernel_name(int kh, int kw, int sh, int sw, int Ho, int dt, bool table, int C, bool groups8) {
  if (table && depthwise_uses_mfma(kh, kw, sh, sw, dt, Ho, C))
    return kh == 5 ? "depthwise_mfma<5x5>" : kh == 7 ? "depthwise_mfma<7x7>" : "depthwise_mfma<9x9>";
  if (kh == 3 && kw == 3 && sh == 2)
    return sw > 2                                     ? "depthwise_strip<3x3,s2>"
           : dt == DT_BF16 && C % 8 == 0 && groups8 ? "depthwise_tiled8<3x3,s2>"
                                                      : "depthwise_tiled<3x3,s2>";
  if (kh == 3 && kw == 3 && sh == 1 && !dw3_tiled_rows(dt, Ho)) return "depthwise_strip<3x3>";
  if (sh == 1 && sw == 1) {
    if (kh == 3 && kw == 3) return dt == DT_BF16 && C % 8 == 0 && groups8 ? "depthwise_tiled8<3x3>" : "depthwise_tiled<3x3>";
    if (kh == kw && (kh == 5 || kh == 7 || kh == 9))
      return kh == 5 ? "depthwise_wave<5x5>" : kh == 7 ? "depthwise_tiled<7x7>" : "depthwise_wave<9x9>";
    if (kh == 1 && (kw == 5 || kw == 7) && Ho == 1) return kw == 5 ? "depthwise_tiled<1x5>" : "depthwise_tiled<1x7>";
  }
  return "depthwise";
}

// ----------------------------------------------------------------- SE gate
// Replaces WGSL `global_mean` + two `conv_single_row` + activation
// (src/gpu/shaders/pool.wgsl:183, conv_single_row.wgsl:84).  Stage 1: each
// block sums a chunk of pixels for all channels (lanes split channels x
// pixel phases, fixed-order LDS reduction).  Stages 2 and 3: the two 1x1
// convs of the squeeze-excitation as wave-per-output products.  The work is
// small and latency-bound: every strided sum issues its loads four at a
// time (then adds them in the same order), and a wave computes its four
// outputs together.

// s += v[k] for k = k0, k0 + step, ... < end, in that order, loads issued
// four at a time.
template <typename T>
__device__ __forceinline__ float4 strided_sum4(float4 s, const T* base, size_t stride, int k0, int end, int step) {
  int k = k0;
  for (; k + 3 * step < end; k += 4 * step) {
    const float4 a = ld4<T>(base + (size_t)k * stride), b = ld4<T>(base + (size_t)(k + step) * stride);
    const float4 c = ld4<T>(base + (size_t)(k + 2 * step) * stride), d = ld4<T>(base + (size_t)(k + 3 * step) * stride);
    s = f4_sum(f4_sum(f4_sum(f4_sum(s, a), b), c), d);
  }
  for (; k < end; k += step) s = f4_sum(s, ld4<T>(base + (size_t)k * stride));
  return s;
}
template <typename T>
__global__ __launch_bounds__(256) void se_partial_kernel(SeParams p, int chunk) {
  __shared__ float4 red[256];
  const T* in = static_cast<const T*>(p.in);
  const int C4 = p.C >> 2;
  const int lanes_p = 256 / C4;
  const int tid = threadIdx.x;
  const int cq = tid % C4;
  const int pl = tid / C4;
  const int n = blockIdx.y;
  const int start = blockIdx.x * chunk;
  const int end = min(start + chunk, p.HW);
  float4 s = f4_zero();
  if (pl < lanes_p) s = strided_sum4<T>(s, in + (size_t)n * p.HW * p.in_ps + cq * 4, p.in_ps, start + pl, end, lanes_p);
  red[tid] = s;
  __syncthreads();
  if (tid < C4) {
    float4 t = red[tid];
    for (int k = 1; k < lanes_p; ++k) t = f4_sum(t, red[k * C4 + tid]);
    *reinterpret_cast<float4*>(p.partial + ((size_t)n * p.P + blockIdx.x) * p.C + tid * 4) = t;
  }
}

// Four wave-per-output matrix-vector products at once: out[q] = sum_i
// W[j_q][i] v[i] with the 64 lanes striding i (coalesced weight rows), each
// lane's terms in increasing i, then a wave reduction.  Rows j_q past
// `rows` are computed on row 0 and ignored by the caller.
__device__ __forceinline__ float4 wave_dot4(const float* __restrict__ w, int j0, int rows, const float* v, int n,
                                            int lane) {
  const float* r0 = w + (size_t)(j0 < rows ? j0 : 0) * n;
  const float* r1 = w + (size_t)(j0 + 1 < rows ? j0 + 1 : 0) * n;
  const float* r2 = w + (size_t)(j0 + 2 < rows ? j0 + 2 : 0) * n;
  const float* r3 = w + (size_t)(j0 + 3 < rows ? j0 + 3 : 0) * n;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  for (int i = lane; i < n; i += 64) {
    const float x = v[i];
    a0 = fmaf(r0[i], x, a0);
    a1 = fmaf(r1[i], x, a1);
    a2 = fmaf(r2[i], x, a2);
    a3 = fmaf(r3[i], x, a3);
  }
  for (int o = 32; o > 0; o >>= 1) {
    a0 += __shfl_xor(a0, o);
    a1 += __shfl_xor(a1, o);
    a2 += __shfl_xor(a2, o);
    a3 += __shfl_xor(a3, o);
  }
  return make_float4(a0, a1, a2, a3);
}

// Stage 2: one block per (image, 16 reduced channels).  The block finishes
// the mean from the partial sums, then each wave computes four outputs of
// the reducing 1x1 conv + bias + ReLU.
__global__ __launch_bounds__(256) void se_reduce_kernel(SeParams p) {
  extern __shared__ float sm[];
  float* mean = sm;                                    // [C]
  float4* red = reinterpret_cast<float4*>(sm + p.C);  // [256]
  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  const int C4 = p.C >> 2;
  const int lanes_p = 256 / C4;
  const int cq = tid % C4, pl = tid / C4;
  float4 s = f4_zero();
  if (pl < lanes_p) s = strided_sum4<float>(s, p.partial + (size_t)n * p.P * p.C + cq * 4, p.C, pl, p.P, lanes_p);
  red[tid] = s;
  __syncthreads();
  if (tid < C4) {
    float4 t = red[tid];
    for (int k = 1; k < lanes_p; ++k) t = f4_sum(t, red[k * C4 + tid]);
    const float count = (float)p.HW;
    mean[tid * 4 + 0] = t.x / count;
    mean[tid * 4 + 1] = t.y / count;
    mean[tid * 4 + 2] = t.z / count;
    mean[tid * 4 + 3] = t.w / count;
  }
  __syncthreads();
  const int wave = tid >> 6, lane = tid & 63;
  const int j0 = blockIdx.y * 16 + wave * 4;
  const float4 acc = wave_dot4(p.w1, j0, p.Cr, mean, p.C, lane);
  const float a[4] = {acc.x, acc.y, acc.z, acc.w};
  if (lane < 4 && j0 + lane < p.Cr) p.hidden[(size_t)n * p.Cr + j0 + lane] = fmaxf(a[lane] + p.b1[j0 + lane], 0.0f);
}

// Stage 3: one block per (image, 16 channels): expanding 1x1 conv + bias and
// the gate activation.
__global__ __launch_bounds__(256) void se_expand_kernel(SeParams p) {
  extern __shared__ float hid[];  // [Cr]
  const int n = blockIdx.x;
  for (int j = threadIdx.x; j < p.Cr; j += 256) hid[j] = p.hidden[(size_t)n * p.Cr + j];
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c0 = blockIdx.y * 16 + wave * 4;
  const float4 acc = wave_dot4(p.w2, c0, p.C, hid, p.Cr, lane);
  const float a[4] = {acc.x, acc.y, acc.z, acc.w};
  if (lane < 4 && c0 + lane < p.C) p.gate[(size_t)n * p.C + c0 + lane] = act_apply(p.gate_act, a[lane] + p.b2[c0 + lane]);
}

// The whole gate of one image in one workgroup (where dependent launches
// cost more than the work): channel means (lanes split channels x pixel
// phases, fixed-order LDS reduction) from the map itself, for small maps, or
// (PARTIALS) from the per-chunk sums left by se_partial or by the depthwise
// that wrote the map; then the reducing and expanding 1x1 convs as in stages
// 2 and 3, 16 waves at a time.
// SMALL (C <= 256, Cr <= 64, the detectors' gates): every weight and bias a
// lane multiplies is loaded before the channel sums, so the two convs wait
// on LDS only (the loop form waits on a load round trip per 64 inputs and per
// bias); the products and their order are those of wave_dot4.
constexpr int kSeSmallC = 256, kSeSmallCr = 64;

template <typename T, bool PARTIALS, bool SMALL>
__device__ __forceinline__ void se_fused_body(const SeParams& p, const int n) {
  extern __shared__ float sm[];
  const int cr4 = (p.Cr + 3) & ~3;
  float* mean = sm;                                          // [C]
  float* hid = sm + p.C;                                     // [Cr]
  float4* red = reinterpret_cast<float4*>(sm + p.C + cr4);  // [1024]
  const T* in = static_cast<const T*>(p.in);
  const int tid = threadIdx.x;
  const int C4 = p.C >> 2;
  const int lanes_p = 1024 / C4;
  const int cq = tid % C4, pl = tid / C4;
  const int wave = tid >> 6, lane = tid & 63;
  constexpr int NI = SMALL ? kSeSmallC / 64 : 1;  // 64-input groups of the reducing conv, passes of the expanding one
  float w1r[NI][4], w2r[NI][4], b2r[NI], b1r = 0.0f;
  if constexpr (SMALL) {
    // Reducing conv: this wave's rows j0 .. j0 + 3 (j0 = 4 wave < 64),
    // inputs lane + 64 it.  Expanding conv: rows 4 wave + 64 it .. + 3,
    // input lane.  Waves without rows load nothing; rows past the matrix
    // read row 0 (ignored), inputs past it read zero.
    const int j0 = wave * 4;
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const int i = lane + 64 * it, c0 = j0 + 64 * it;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r1 = j0 + q < p.Cr ? j0 + q : 0, r2 = c0 + q < p.C ? c0 + q : 0;
        w1r[it][q] = j0 < p.Cr && i < p.C ? p.w1[(size_t)r1 * p.C + i] : 0.0f;
        w2r[it][q] = c0 < p.C && lane < p.Cr ? p.w2[(size_t)r2 * p.Cr + lane] : 0.0f;
      }
      b2r[it] = lane < 4 && c0 + lane < p.C ? p.b2[c0 + lane] : 0.0f;
    }
    if (lane < 4 && j0 + lane < p.Cr) b1r = p.b1[j0 + lane];
  }
  float4 s = f4_zero();
  if (pl < lanes_p) {
    if constexpr (PARTIALS)
      s = strided_sum4<float>(s, p.partial + (size_t)n * p.P * p.C + cq * 4, p.C, pl, p.P, lanes_p);
    else
      s = strided_sum4<T>(s, in + (size_t)n * p.HW * p.in_ps + cq * 4, p.in_ps, pl, p.HW, lanes_p);
  }
  red[tid] = s;
  __syncthreads();
  // Two-level sum of the lanes_p phases of each channel quad: G partial
  // sums of every G-th phase (in place: slot g of quad cq is read only by
  // its own thread), then the G partials in order.
  const int G = lanes_p < 16 ? lanes_p : 16;
  if (tid < G * C4) {
    float4 t = red[tid];
    for (int k = pl + G; k < lanes_p; k += G) t = f4_sum(t, red[k * C4 + cq]);
    red[tid] = t;
  }
  __syncthreads();
  if (tid < C4) {
    float4 t = red[tid];
    for (int k = 1; k < G; ++k) t = f4_sum(t, red[k * C4 + tid]);
    const float count = (float)p.HW;
    mean[tid * 4 + 0] = t.x / count;
    mean[tid * 4 + 1] = t.y / count;
    mean[tid * 4 + 2] = t.z / count;
    mean[tid * 4 + 3] = t.w / count;
  }
  __syncthreads();
  if constexpr (SMALL) {
    const int j0 = wave * 4;
    if (j0 < p.Cr) {
      float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int it = 0; it < NI; ++it) {
        const int i = lane + 64 * it;
        if (i < p.C) {  // the terms wave_dot4 takes, in its order
          const float x = mean[i];
#pragma unroll
          for (int q = 0; q < 4; ++q) a[q] = fmaf(w1r[it][q], x, a[q]);
        }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1)
#pragma unroll
        for (int q = 0; q < 4; ++q) a[q] += __shfl_xor(a[q], o);
      const float mine = lane == 0 ? a[0] : lane == 1 ? a[1] : lane == 2 ? a[2] : a[3];
      if (lane < 4 && j0 + lane < p.Cr) hid[j0 + lane] = fmaxf(mine + b1r, 0.0f);
    }
    __syncthreads();
    const float x = lane < p.Cr ? hid[lane] : 0.0f;
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const int c0 = wave * 4 + 64 * it;
      if (c0 >= p.C) break;
      float a[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) a[q] = lane < p.Cr ? fmaf(w2r[it][q], x, 0.0f) : 0.0f;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1)
#pragma unroll
        for (int q = 0; q < 4; ++q) a[q] += __shfl_xor(a[q], o);
      const float mine = lane == 0 ? a[0] : lane == 1 ? a[1] : lane == 2 ? a[2] : a[3];
      if (lane < 4 && c0 + lane < p.C) p.gate[(size_t)n * p.C + c0 + lane] = act_apply(p.gate_act, mine + b2r[it]);
    }
    return;
  }
  for (int j0 = wave * 4; j0 < p.Cr; j0 += 64) {
    const float4 acc = wave_dot4(p.w1, j0, p.Cr, mean, p.C, lane);
    const float a[4] = {acc.x, acc.y, acc.z, acc.w};
    if (lane < 4 && j0 + lane < p.Cr) hid[j0 + lane] = fmaxf(a[lane] + p.b1[j0 + lane], 0.0f);
  }
  __syncthreads();
  for (int c0 = wave * 4; c0 < p.C; c0 += 64) {
    const float4 acc = wave_dot4(p.w2, c0, p.C, hid, p.Cr, lane);
    const float a[4] = {acc.x, acc.y, acc.z, acc.w};
    if (lane < 4 && c0 + lane < p.C)
      p.gate[(size_t)n * p.C + c0 + lane] = act_apply(p.gate_act, a[lane] + p.b2[c0 + lane]);
  }
}

template <typename T, bool PARTIALS, bool SMALL>
__global__ __launch_bounds__(1024) void se_fused_kernel(SeParams p) {
  se_fused_body<T, PARTIALS, SMALL>(p, blockIdx.x);
}

// Several gates from given partial sums, one per grid row (the cases index
// the parameter array with constants, so it stays in kernel arguments).
template <bool SMALL>
__global__ __launch_bounds__(1024) void se_multi_kernel(SeMulti m) {
  switch (blockIdx.y) {
    case 0: se_fused_body<float, true, SMALL>(m.p[0], blockIdx.x); break;
    case 1: se_fused_body<float, true, SMALL>(m.p[1], blockIdx.x); break;
    case 2: se_fused_body<float, true, SMALL>(m.p[2], blockIdx.x); break;
    default: se_fused_body<float, true, SMALL>(m.p[3], blockIdx.x); break;
  }
}

bool se_fused(const SeParams& p) {
  const size_t es = p.dt == DT_BF16 ? 2 : 4;
  return p.C % 4 == 0 && p.C <= 4096 && (size_t)p.HW * p.C * es <= (256u << 10) &&
         (size_t)p.C * p.Cr * 2 * sizeof(float) <= (128u << 10);
}

// From the partial sums: one workgroup per image does the means and both
// 1x1 convs while their weights are small (one CU pulls them from L2 at a
// few hundred bytes per cycle); otherwise the two stages spread the weight
// rows over many workgroups.
static bool se_gate_one_block(const SeParams& p) {
  return p.C <= 4096 && (size_t)p.C * p.Cr * 2 * sizeof(float) <= (128u << 10);
}

void launch_se_from_partials(const SeParams& p, hipStream_t s) {
  if (se_gate_one_block(p)) {
    const size_t lds = ((size_t)p.C + ((p.Cr + 3) & ~3)) * sizeof(float) + 1024 * sizeof(float4);
    if (p.C <= kSeSmallC && p.Cr <= kSeSmallCr)
      hipLaunchKernelGGL((se_fused_kernel<float, true, true>), dim3(p.N), dim3(1024), lds, s, p);
    else
      hipLaunchKernelGGL((se_fused_kernel<float, true, false>), dim3(p.N), dim3(1024), lds, s, p);
    return;
  }
  size_t lds = (size_t)p.C * sizeof(float) + 256 * sizeof(float4);
  hipLaunchKernelGGL(se_reduce_kernel, dim3(p.N, (p.Cr + 15) / 16), dim3(256), lds, s, p);
  hipLaunchKernelGGL(se_expand_kernel, dim3(p.N, (p.C + 15) / 16), dim3(256), (size_t)p.Cr * sizeof(float), s, p);
}

static size_t se_one_block_lds(const SeParams& p) {
  return ((size_t)p.C + ((p.Cr + 3) & ~3)) * sizeof(float) + 1024 * sizeof(float4);
}

int se_multi_kind(const SeParams& p) {
  if (!se_gate_one_block(p) || p.C % 4 || p.P < 1) return 0;
  return p.C <= kSeSmallC && p.Cr <= kSeSmallCr ? 1 : 2;
}

void launch_se_multi(const SeMulti& m, hipStream_t s) {
  if (m.count < 1 || m.count > kSeMultiMax) throw std::runtime_error("launch_se_multi: 1 to 4 gates");
  const int kind = se_multi_kind(m.p[0]);
  size_t lds = 0;
  for (int i = 0; i < m.count; ++i) {
    if (se_multi_kind(m.p[i]) != kind || kind == 0 || m.p[i].N != m.p[0].N)
      throw std::runtime_error("launch_se_multi: gates of different kinds or image counts");
    lds = std::max(lds, se_one_block_lds(m.p[i]));
  }
  const dim3 grid((unsigned)m.p[0].N, (unsigned)m.count);
  if (kind == 1)
    hipLaunchKernelGGL(se_multi_kernel<true>, grid, dim3(1024), lds, s, m);
  else
    hipLaunchKernelGGL(se_multi_kernel<false>, grid, dim3(1024), lds, s, m);
}

void launch_se(const SeParams& p, hipStream_t s) {
  if (se_fused(p)) {
    const size_t lds = ((size_t)p.C + ((p.Cr + 3) & ~3)) * sizeof(float) + 1024 * sizeof(float4);
    if (p.C <= kSeSmallC && p.Cr <= kSeSmallCr)
      DISPATCH_DT(p.dt, hipLaunchKernelGGL((se_fused_kernel<T, false, true>), dim3(p.N), dim3(1024), lds, s, p));
    else
      DISPATCH_DT(p.dt, hipLaunchKernelGGL((se_fused_kernel<T, false, false>), dim3(p.N), dim3(1024), lds, s, p));
    return;
  }
  int chunk = (p.HW + p.P - 1) / p.P;
  DISPATCH_DT(p.dt, hipLaunchKernelGGL(se_partial_kernel<T>, dim3(p.P, p.N), dim3(256), 0, s, p, chunk));
  launch_se_from_partials(p, s);
}

// ----------------------------------------------------------------- layout
template <typename T>
__global__ void nchw_to_nhwc4_kernel(const float* in, T* out, int N, int H, int W) {
  long idx = (long)blockIdx.x * 256 + threadIdx.x;
  long plane = (long)H * W;
  if (idx >= (long)N * plane) return;
  int n = (int)(idx / plane);
  long i = idx - n * plane;
  const float* src = in + (size_t)n * 3 * plane + i;
  st4<T>(out + (size_t)idx * 4, make_float4(src[0], src[plane], src[2 * plane], 0.0f));
}

void launch_nchw_to_nhwc4(const float* in, void* out, int N, int H, int W, int dt, hipStream_t s) {
  DISPATCH_DT(dt, hipLaunchKernelGGL(nchw_to_nhwc4_kernel<T>, dim3(blocks_for((long)N * H * W)), dim3(256), 0, s, in,
                                     static_cast<T*>(out), N, H, W));
}

// ----------------------------------------------------------------- pools
// Max pool 2x2 / stride 1 / pads (0,0,1,1) of the large stem
// (src/cpu/model.rs:689, src/cpu/ops.rs:1520-1535); fmaxf ignores NaN like
// f32::max.
// 2x2 stride-1 max pool whose windows past the bottom / right edge are
// clipped (pads 0,0,1,1; NaN-ignoring max as f32::max).  A lane computes
// MP_R output rows of one pixel column and four channels: it loads the
// MP_R + 1 input rows it needs (two pixels each) once, all before its first
// store, and reuses each row's pair maximum for the two outputs that share it
// (every input row is read by one strip, plus the strip above at its edge,
// instead of by four windows).
constexpr int MP_R = 4;

template <typename T>
__global__ void maxpool_same_kernel(const T* __restrict__ in, int N, int H, int W, int C, int in_ps,
                                    T* __restrict__ out, int out_ps) {
  const int C4 = C >> 2;
  const int strips = (H + MP_R - 1) / MP_R;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  const long total = (long)N * strips * W * C4;
  if (idx >= total) return;
  const int c = (int)(idx % C4) * 4;
  long t = idx / C4;
  const int x = (int)(t % W);
  t /= W;
  const int s = (int)(t % strips);
  const int n = (int)(t / strips);
  const int y0 = s * MP_R;
  const bool right = x + 1 < W;
  float4 rm[MP_R + 1];  // pair maximum of rows y0 .. y0 + MP_R (rows past H unused)
#pragma unroll
  for (int r = 0; r <= MP_R; ++r) {
    const int y = y0 + r;
    rm[r] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    if (y < H) {
      const T* px = in + ((size_t)(n * H + y) * W + x) * in_ps + c;
      const float4 a = ld4<T>(px);
      const float4 b = right ? ld4<T>(px + in_ps) : a;
      rm[r] = make_float4(fmaxf(a.x, b.x), fmaxf(a.y, b.y), fmaxf(a.z, b.z), fmaxf(a.w, b.w));
    }
  }
#pragma unroll
  for (int r = 0; r < MP_R; ++r) {
    const int y = y0 + r;
    if (y >= H) break;
    const float4 a = rm[r], b = rm[r + 1];  // rm[r + 1] is -inf past the last row
    st4<T>(out + ((size_t)(n * H + y) * W + x) * out_ps + c,
           make_float4(fmaxf(a.x, b.x), fmaxf(a.y, b.y), fmaxf(a.z, b.z), fmaxf(a.w, b.w)));
  }
}

void launch_maxpool_same(const void* in, int N, int H, int W, int C, int in_ps, void* out, int out_ps, int dt,
                         hipStream_t s) {
  const long total = (long)N * ((H + MP_R - 1) / MP_R) * W * (C / 4);
  DISPATCH_DT(dt, hipLaunchKernelGGL(maxpool_same_kernel<T>, dim3(blocks_for(total)), dim3(256), 0, s,
                                     static_cast<const T*>(in), N, H, W, C, in_ps, static_cast<T*>(out), out_ps));
}

// Average pool [3,2] / [3,2], no padding, count_include_pad = false
// (src/cpu/ops.rs:1537-1604): the six taps are summed in row-major order.
template <typename T>
__global__ void avgpool32_kernel(const T* in, int N, int H, int W, int C, int in_ps, T* out, int Ho, int Wo) {
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
    for (int kx = 0; kx < 2; ++kx)
      s = f4_sum(s, ld4<T>(in + ((size_t)(n * H + oy * 3 + ky) * W + ox * 2 + kx) * in_ps + c));
  st4<T>(out + (size_t)pix * C + c, make_float4(s.x / 6.0f, s.y / 6.0f, s.z / 6.0f, s.w / 6.0f));
}

void launch_avgpool32(const void* in, int N, int H, int W, int C, int in_ps, void* out, int Ho, int Wo, int dt,
                      hipStream_t s) {
  long total = (long)N * Ho * Wo * (C / 4);
  DISPATCH_DT(dt, hipLaunchKernelGGL(avgpool32_kernel<T>, dim3(blocks_for(total)), dim3(256), 0, s,
                                     static_cast<const T*>(in), N, H, W, C, in_ps, static_cast<T*>(out), Ho, Wo));
}

// ----------------------------------------------------------------- FPN
// Residual squeeze-excitation output x + x*g (src/cpu/model.rs:1138-1142,
// :1188-1194), fused with the top-down nearest-upsample add
// (upsample_add_nchw, :1265-1320) or with the upsample-and-concat write
// (upsample_and_cat_nchw, :1322-1417): each input pixel is written as a
// rep x rep block into its channel slice of the concat tensor.
template <typename T>
__device__ __forceinline__ void gate_residual_at(long idx, const T* in, int N, int H, int W, int C, int in_ps,
                                                 const float* gate, const T* upper, int up_ps, T* out, int out_ps,
                                                 int rep) {
  const int C4 = C >> 2;
  long total = (long)N * H * W * C4;
  if (idx >= total) return;
  int c = (int)(idx % C4) * 4;
  long pix = idx / C4;
  int x = (int)(pix % W);
  long t = pix / W;
  int y = (int)(t % H);
  int n = (int)(t / H);
  float4 v = ld4<T>(in + (size_t)pix * in_ps + c);
  float4 g = *reinterpret_cast<const float4*>(gate + (size_t)n * C + c);
  v = make_float4(residual_mul(v.x, g.x), residual_mul(v.y, g.y), residual_mul(v.z, g.z), residual_mul(v.w, g.w));
  if (upper) {
    int uh = H / 2, uw = W / 2;
    v = f4_sum(v, ld4<T>(upper + ((size_t)(n * uh + y / 2) * uw + x / 2) * up_ps + c));
  }
  if (rep == 1) {
    st4<T>(out + (size_t)pix * out_ps + c, v);
  } else {
    int OW = W * rep;
    for (int dy = 0; dy < rep; ++dy) {
      T* row = out + ((size_t)(n * H * rep + y * rep + dy) * OW + (size_t)x * rep) * out_ps + c;
      for (int dx = 0; dx < rep; ++dx) st4<T>(row + (size_t)dx * out_ps, v);
    }
  }
}

template <typename T>
__global__ void gate_residual_kernel(const T* in, int N, int H, int W, int C, int in_ps, const float* gate,
                                     const T* upper, int up_ps, T* out, int out_ps, int rep) {
  gate_residual_at<T>((long)blockIdx.x * 256 + threadIdx.x, in, N, H, W, C, in_ps, gate, upper, up_ps, out, out_ps,
                      rep);
}

// Several gate_residual writes in one launch: block b belongs to the last
// part whose first block is <= b (constant indices into the kernel
// arguments, as in se_multi_kernel).
template <typename T>
__global__ void gate_residual_multi_kernel(GateResidualMulti m, int first1, int first2, int first3) {
  const int b = blockIdx.x;
  const int i = (b >= first1) + (b >= first2) + (b >= first3);
  const int first = i == 0 ? 0 : i == 1 ? first1 : i == 2 ? first2 : first3;
  const long idx = (long)(b - first) * 256 + threadIdx.x;
  auto run = [&](const GateResidualPart& q) {
    gate_residual_at<T>(idx, static_cast<const T*>(q.in), m.N, q.H, q.W, q.C, q.in_ps, q.gate, nullptr, 0,
                        static_cast<T*>(q.out), q.out_ps, q.rep);
  };
  switch (i) {
    case 0: run(m.part[0]); break;
    case 1: run(m.part[1]); break;
    case 2: run(m.part[2]); break;
    default: run(m.part[3]); break;
  }
}

void launch_gate_residual(const void* in, int N, int H, int W, int C, int in_ps, const float* gate,
                          const void* upper, int up_ps, void* out, int out_ps, int rep, int dt, hipStream_t s) {
  long total = (long)N * H * W * (C / 4);
  DISPATCH_DT(dt, hipLaunchKernelGGL(gate_residual_kernel<T>, dim3(blocks_for(total)), dim3(256), 0, s,
                                     static_cast<const T*>(in), N, H, W, C, in_ps, gate,
                                     static_cast<const T*>(upper), up_ps, static_cast<T*>(out), out_ps, rep));
}

void launch_gate_residual_multi(const GateResidualMulti& m, hipStream_t s) {
  if (m.count < 1 || m.count > 4) throw std::runtime_error("launch_gate_residual_multi: 1 to 4 parts");
  int first[4] = {0, INT32_MAX, INT32_MAX, INT32_MAX};
  long blocks = 0;
  for (int i = 0; i < m.count; ++i) {
    first[i] = (int)blocks;
    blocks += blocks_for((long)m.N * m.part[i].H * m.part[i].W * (m.part[i].C / 4));
  }
  DISPATCH_DT(m.dt, hipLaunchKernelGGL(gate_residual_multi_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s, m,
                                       first[1], first[2], first[3]));
}

// SE gate applied to a whole tensor: out = x * g[n, c] rounded to the
// storage type, the value the consumer conv would otherwise form while
// gathering A (the SE multiply of src/cpu/model.rs:1138-1142).
template <typename T>
__global__ void scale_channels_kernel(const T* in, long pixels, int HW, int C, int in_ps, const float* gate, T* out) {
  const int C4 = C >> 2;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= pixels * C4) return;
  const int c = (int)(idx % C4) * 4;
  const long pix = idx / C4;
  const float4 v = ld4<T>(in + (size_t)pix * in_ps + c);
  const float4 g = *reinterpret_cast<const float4*>(gate + (size_t)(pix / HW) * C + c);
  st4<T>(out + (size_t)pix * C + c, make_float4(v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w));
}

void launch_scale_channels(const void* in, int N, int HW, int C, int in_ps, const float* gate, void* out, int dt,
                           hipStream_t s) {
  const long pixels = (long)N * HW;
  DISPATCH_DT(dt, hipLaunchKernelGGL(scale_channels_kernel<T>, dim3(blocks_for(pixels * (C / 4))), dim3(256), 0, s,
                                     static_cast<const T*>(in), pixels, HW, C, in_ps, gate, static_cast<T*>(out)));
}

// ----------------------------------------------------------------- DB head
// Replaces WGSL `detector_head` / `deconv_phase` + `deconv_final`
// (src/gpu/shaders/detector_head.wgsl:52, deconv_phase.wgsl:105,
// deconv_final.wgsl:52).  Per input pixel at H/4 x W/4: conv_up (2x2 s2,
// BN folded, +bias, ReLU) then conv_final (2x2 s2 to one channel, +bias)
// and sigmoid (src/cpu/model.rs:1516-1520), 16 probabilities per lane.
// Weights: wu [c][o][4] (IOHW, folded), bu [o], wf [o][4].
template <typename T, int CH>
__global__ __launch_bounds__(256) void db_head_up_kernel(const T* in, int N, int H, int W, int in_ps,
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
  const T* src = in + (size_t)idx * in_ps;
#pragma unroll
  for (int c = 0; c < CH; c += 4) {
    float4 v = ld4<T>(src + c);
    xin[c] = v.x;
    xin[c + 1] = v.y;
    xin[c + 2] = v.z;
    xin[c + 3] = v.w;
  }
  const int OW = 4 * W;
#pragma unroll 1
  for (int tap = 0; tap < 4; ++tap) {
    float f[4] = {0.f, 0.f, 0.f, 0.f};
    // Rolled over the hidden channels: only the input pixel and one hidden
    // value are live, which keeps the kernel free of spills for every CH.
#pragma unroll 1
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
    float2 top = make_float2(act_apply(ACT_SIGMOID, f[0] + bf), act_apply(ACT_SIGMOID, f[1] + bf));
    float2 bot = make_float2(act_apply(ACT_SIGMOID, f[2] + bf), act_apply(ACT_SIGMOID, f[3] + bf));
    *reinterpret_cast<float2*>(o0) = top;
    *reinterpret_cast<float2*>(o0 + OW) = bot;
  }
}

template <typename T>
static void launch_db_typed(const void* in, int N, int H, int W, int Ch, int in_ps, const float* wu, const float* bu,
                            const float* wf, float bf, float* out, hipStream_t s) {
  dim3 grid(blocks_for((long)N * H * W));
  const T* x = static_cast<const T*>(in);
  switch (Ch) {
    case 16: hipLaunchKernelGGL((db_head_up_kernel<T, 16>), grid, dim3(256), 0, s, x, N, H, W, in_ps, wu, bu, wf, bf, out); break;
    case 24: hipLaunchKernelGGL((db_head_up_kernel<T, 24>), grid, dim3(256), 0, s, x, N, H, W, in_ps, wu, bu, wf, bf, out); break;
    case 64: hipLaunchKernelGGL((db_head_up_kernel<T, 64>), grid, dim3(256), 0, s, x, N, H, W, in_ps, wu, bu, wf, bf, out); break;
    default: break;  // rejected by the planner
  }
}

void launch_db_head_up(const void* in, int N, int H, int W, int Ch, int in_ps, const float* wu, const float* bu,
                       const float* wf, float bf, float* out, int dt, hipStream_t s) {
  DISPATCH_DT(dt, launch_db_typed<T>(in, N, H, W, Ch, in_ps, wu, bu, wf, bf, out, s));
}

// ----------------------------------------------------------------- LayerNorm
// Replaces WGSL `layer_norm` (src/gpu/shaders/layer_norm.wgsl:55); formula
// of layer_norm_in_place (src/cpu/kernels/mod.rs:2288-2313): two-pass mean
// and variance, out = (x - mean) * (inv_std * w) + b; one wave per row.
template <typename T>
__global__ __launch_bounds__(256) void layer_norm_kernel(const T* in, int rows, int C, const float* w, const float* b,
                                                         float eps, const T* res, T* out) {
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const T* x = in + (size_t)row * C;
  float s = 0.0f;
  for (int c = lane; c < C; c += 64) s += ld1<T>(x + c);
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  float mean = s / (float)C;
  float v = 0.0f;
  for (int c = lane; c < C; c += 64) {
    float d = ld1<T>(x + c) - mean;
    v = fmaf(d, d, v);
  }
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  float var = v / (float)C;
  float inv = 1.0f / sqrtf(var + eps);
  T* y = out + (size_t)row * C;
  for (int c = lane; c < C; c += 64) {
    float r = fmaf(ld1<T>(x + c) - mean, inv * w[c], b[c]);
    if (res) r = r + ld1<T>(res + (size_t)row * C + c);
    st1<T>(y + c, r);
  }
}

void launch_layer_norm(const void* in, int rows, int C, const float* w, const float* b, float eps, const void* res,
                       void* out, int dt, hipStream_t s) {
  DISPATCH_DT(dt, hipLaunchKernelGGL(layer_norm_kernel<T>, dim3(blocks_for(rows, 4)), dim3(256), 0, s,
                                     static_cast<const T*>(in), rows, C, w, b, eps, static_cast<const T*>(res),
                                     static_cast<T*>(out)));
}

// ----------------------------------------------------------------- attention
// Replaces WGSL `attention_scores` + `attention_context`
// (src/gpu/shaders/attention.wgsl:62, :151); RecAttention::forward
// (src/cpu/model.rs:1703-1725): qkv rows laid out [3, heads, hd];
// scores = (q . k) * hd^-0.5, softmax over the keys, context = P v.
//
// The softmax is computed online (running maximum and running sum, rescaled
// when the maximum grows), so no score row is ever held whole and the
// sequence length has no bound: a workgroup owns one (image, head) and 64
// queries, four lanes per query; key and value rows stream through LDS 64 at
// a time, each lane scoring every fourth key of a tile and folding them into
// its own (max, sum, context) state; the four states of a query are merged
// with lane shuffles at the end.  HD is the head dimension rounded up to the
// register tile (16, 24 or 32); the padding lanes of q, k and v are zero.
constexpr int FA_Q = 64;
constexpr int FA_K = 64;

template <typename T, int HD>
__global__ __launch_bounds__(256) void flash_attention_kernel(const T* qkv, int T_, int hidden, int heads,
                                                              float scale, T* out) {
  __shared__ float ks[FA_K * HD];
  __shared__ float vs[FA_K * HD];
  const int bh = blockIdx.x;
  const int b = bh / heads, h = bh - b * heads;
  const int hd = hidden / heads;
  const int qi = threadIdx.x >> 2, sub = threadIdx.x & 3;
  const int t = blockIdx.y * FA_Q + qi;
  const size_t stride = (size_t)3 * hidden;
  const T* base = qkv + (size_t)b * T_ * stride + h * hd;
  const bool valid = t < T_;
  float q[HD], acc[HD];
#pragma unroll
  for (int d = 0; d < HD; ++d) {
    q[d] = valid && d < hd ? ld1<T>(base + (size_t)t * stride + d) : 0.0f;
    acc[d] = 0.0f;
  }
  float m = -INFINITY, l = 0.0f;
  for (int k0 = 0; k0 < T_; k0 += FA_K) {
    const int nk = min(FA_K, T_ - k0);
    __syncthreads();  // the previous tile is no longer read
    for (int i = threadIdx.x; i < FA_K * HD; i += 256) {
      const int j = i / HD, d = i - j * HD;
      const bool in = j < nk && d < hd;
      const T* row = base + (size_t)(k0 + j) * stride;
      ks[i] = in ? ld1<T>(row + hidden + d) : 0.0f;
      vs[i] = in ? ld1<T>(row + 2 * hidden + d) : 0.0f;
    }
    __syncthreads();
    float sc[FA_K / 4];
    float cm = -INFINITY;
#pragma unroll
    for (int i = 0; i < FA_K / 4; ++i) {
      const int j = sub + 4 * i;
      const float* kr = ks + j * HD;
      float a = 0.0f;
#pragma unroll
      for (int d = 0; d < HD; ++d) a = fmaf(q[d], kr[d], a);
      sc[i] = j < nk ? a * scale : -INFINITY;
      cm = fmaxf(cm, sc[i]);
    }
    const float mn = fmaxf(m, cm);
    if (mn > -INFINITY) {
      const float corr = fast_exp(m - mn);  // 0 while nothing was folded (m = -inf)
      l *= corr;
#pragma unroll
      for (int d = 0; d < HD; ++d) acc[d] *= corr;
#pragma unroll
      for (int i = 0; i < FA_K / 4; ++i) {
        const float pr = fast_exp(sc[i] - mn);  // 0 for keys past the sequence
        l += pr;
        const float* vr = vs + (sub + 4 * i) * HD;
#pragma unroll
        for (int d = 0; d < HD; ++d) acc[d] = fmaf(pr, vr[d], acc[d]);
      }
      m = mn;
    }
  }
  // Merge the four partial states of this query (lanes 4q .. 4q + 3).
#pragma unroll
  for (int o = 1; o < 4; o <<= 1) {
    const float m2 = __shfl_xor(m, o), l2 = __shfl_xor(l, o);
    const float mn = fmaxf(m, m2);
    const float c1 = m == -INFINITY ? 0.0f : fast_exp(m - mn);
    const float c2 = m2 == -INFINITY ? 0.0f : fast_exp(m2 - mn);
    l = l * c1 + l2 * c2;
#pragma unroll
    for (int d = 0; d < HD; ++d) acc[d] = acc[d] * c1 + __shfl_xor(acc[d], o) * c2;
    m = mn;
  }
  if (valid) {
    const float r = 1.0f / l;
    T* o = out + ((size_t)b * T_ + t) * hidden + h * hd;
#pragma unroll
    for (int d = 0; d < HD; ++d)
      if ((d & 3) == sub && d < hd) st1<T>(o + d, acc[d] * r);
  }
}

int attention_head_tile(int hd) { return hd <= 16 ? 16 : hd <= 24 ? 24 : hd <= 32 ? 32 : 0; }

void launch_attention(const void* qkv, int B, int T_, int hidden, int heads, void* out, int dt, hipStream_t s) {
  const int hd = hidden / heads;
  const float scale = powf((float)hd, -0.5f);
  dim3 grid(B * heads, (T_ + FA_Q - 1) / FA_Q);
#define FA_LAUNCH(HDV)                                                                                     \
  DISPATCH_DT(dt, hipLaunchKernelGGL((flash_attention_kernel<T, HDV>), grid, dim3(256), 0, s,             \
                                     static_cast<const T*>(qkv), T_, hidden, heads, scale, static_cast<T*>(out)))
  switch (attention_head_tile(hd)) {
    case 16: FA_LAUNCH(16); break;
    case 24: FA_LAUNCH(24); break;
    default: FA_LAUNCH(32); break;
  }
#undef FA_LAUNCH
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
  for (int i = threadIdx.x; i < cols; i += blockDim.x) s += fast_exp(row[i] - m);
  s = block_reduce(s, red, false);
  float rcp = 1.0f / s;
  for (int i = threadIdx.x; i < cols; i += blockDim.x) row[i] = fast_exp(row[i] - m) * rcp;
}

// Even row lengths up to 2 * NT * PER (the recognizers' 6.9k-18.7k
// classes): the row is read once into registers (PER float2 per thread;
// rows are 8-byte aligned), so it crosses HBM once each way instead of being
// read for the maximum, again for the sum and again for the store.  NT = 1024
// threads for few rows (latency); 256 for 2048 rows or more, so that other
// rows load while one block reduces (50 VGPRs at PER = 16, eight blocks per
// CU; 93 at PER = 40, five).
template <int PER, int NT = 1024>
__global__ __launch_bounds__(NT) void softmax_rows_reg_kernel(float* x, int cols) {
  __shared__ float red[16];
  // The row through a buffer resource: the lane's byte offset 8 * tid in one
  // register and chunk j's offset 8 * NT * j in a scalar one, so no 64-bit
  // address per chunk stays live from the loads to the stores.  Accesses are
  // limited to the row by the lane conditions (none rely on range checks).
  const int32x4_t row = buffer_resource(x + (size_t)blockIdx.x * cols, (unsigned)cols * 4u);
  const int n2 = cols >> 1;
  const int vo = (int)threadIdx.x * 8;
  float2 v[PER];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    v[j] = make_float2(-INFINITY, -INFINITY);
    if ((int)threadIdx.x + j * NT < n2) {
      const f32x2v u = llvm_raw_buffer_load_v2f32(row, vo, j * NT * 8, 0);
      v[j] = make_float2(u.x, u.y);
    }
    m = fmaxf(m, fmaxf(v[j].x, v[j].y));
  }
  m = block_reduce(m, red, true);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (threadIdx.x + j * NT < n2) {
      v[j].x = fast_exp(v[j].x - m);
      v[j].y = fast_exp(v[j].y - m);
      s += v[j].x + v[j].y;
    }
  }
  s = block_reduce(s, red, false);
  const float rcp = 1.0f / s;
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if ((int)threadIdx.x + j * NT < n2) {
      const f32x2v o = {v[j].x * rcp, v[j].y * rcp};
      llvm_raw_buffer_store_v2f32(o, row, vo, j * NT * 8, 0);
    }
}

void launch_softmax_rows(float* x, long rows, int cols, hipStream_t s) {
  const int per = (cols / 2 + 1023) / 1024;
  const bool even = cols % 2 == 0 && reinterpret_cast<uintptr_t>(x) % 8 == 0;
  const dim3 grid((unsigned)rows), block(1024);
  const int per256 = (cols / 2 + 255) / 256;
  if (even && rows >= 2048 && per256 <= 16)
    hipLaunchKernelGGL((softmax_rows_reg_kernel<16, 256>), grid, dim3(256), 0, s, x, cols);
  else if (even && rows >= 2048 && per256 <= 40)
    hipLaunchKernelGGL((softmax_rows_reg_kernel<40, 256>), grid, dim3(256), 0, s, x, cols);
  else if (even && per <= 4)
    hipLaunchKernelGGL(softmax_rows_reg_kernel<4>, grid, block, 0, s, x, cols);
  else if (even && per <= 10)
    hipLaunchKernelGGL(softmax_rows_reg_kernel<10>, grid, block, 0, s, x, cols);
  else if (even && per <= 16)
    hipLaunchKernelGGL(softmax_rows_reg_kernel<16>, grid, block, 0, s, x, cols);
  else
    hipLaunchKernelGGL(softmax_rows_kernel, grid, block, 0, s, x, cols);
}

// ------------------------------------------------------------ greedy CTC merge
// Second half of the classifier's greedy-CTC epilogue.  Partials are planes
// [3][n_tiles][M] (max, sum exp, last argmax).  A block covers 64 rows with
// four lanes per row, each folding every fourth column tile (a wave reads 64
// consecutive rows of one tile: coalesced); the four are merged through LDS.
// The argmax's softmax value is exp(0) / sum = 1 / sum.
__global__ __launch_bounds__(256) void ctc_merge_kernel(const float* part, int M, int n_tiles, float* out) {
  __shared__ float sm[4][64], ss[4][64];
  __shared__ int si[4][64];
  const int r = threadIdx.x & 63, split = threadIdx.x >> 6;
  const int m = blockIdx.x * 64 + r;
  float mx = -INFINITY, sum = 0.0f;
  int idx = -1;
  if (m < M) {
    const size_t plane = (size_t)n_tiles * M;
    for (int j = split; j < n_tiles; j += 4) {
      const size_t at = (size_t)j * M + m;
      lse_merge(mx, sum, idx, part[at], part[plane + at], (int)part[2 * plane + at]);
    }
  }
  sm[split][r] = mx;
  ss[split][r] = sum;
  si[split][r] = idx;
  __syncthreads();
  if (split == 0 && m < M) {
#pragma unroll
    for (int k = 1; k < 4; ++k) lse_merge(mx, sum, idx, sm[k][r], ss[k][r], si[k][r]);
    out[2 * (size_t)m] = (float)idx;
    out[2 * (size_t)m + 1] = 1.0f / sum;
  }
}

void launch_ctc_merge(const float* part, int M, int n_tiles, float* out, hipStream_t s) {
  hipLaunchKernelGGL(ctc_merge_kernel, dim3((unsigned)((M + 63) / 64)), dim3(256), 0, s, part, M, n_tiles, out);
}

// ----------------------------------------------------------------- preprocess
// The reference CPU preprocessing (src/preprocess/kernels.rs:94-170): quad
// bilinear source point, clamped; bilinear RGB rounded to an integer and
// clamped; v * (1/(255 std)) - mean/std as BGR planes; zero past
// content_width.  Contraction is off so every product and sum rounds as in
// the reference.
// NHWC4 (T non-void): the pixel's four channels (B, G, R, 0) go straight to
// the model input in its storage type, the values the fp32 planes would
// hold after nchw_to_nhwc4_kernel.
template <typename T>
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
  if constexpr (std::is_void_v<T>) {
    float* o = p.out + (size_t)n * 3 * plane + r;
    o[0] = b;
    o[plane] = g;
    o[2 * plane] = rr;
  } else {
    st4<T>(static_cast<T*>(p.nhwc4) + (size_t)idx * 4, make_float4(b, g, rr, 0.0f));
  }
}

void launch_preprocess(const PreParams& p, hipStream_t s) {
  long total = (long)p.N * p.ch * p.cw;
  if (!p.nhwc4)
    hipLaunchKernelGGL(preprocess_kernel<void>, dim3(blocks_for(total)), dim3(256), 0, s, p);
  else
    DISPATCH_DT(p.dt, hipLaunchKernelGGL(preprocess_kernel<T>, dim3(blocks_for(total)), dim3(256), 0, s, p));
}

}  // namespace ppocr
