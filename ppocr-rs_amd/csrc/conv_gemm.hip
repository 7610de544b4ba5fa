// Implicit-GEMM convolution on the CDNA4 fp32 matrix cores.
//
// Replaces the reference's WGSL `conv`, `conv_medium_linear`,
// `conv_single_row`, `conv_spatial_m32`, `conv_2x2_direct`,
// `conv_3x3_stride2_direct`, `conv_3x3_direct`, `deconv2x2`, `deconv_phase`
// (src/gpu/shaders/*.wgsl; kernel selection src/gpu/runtime.rs:699-949) with
// one tiled kernel:
//   * M = output pixels (NHWC rows), N = output channels, K = kh*kw*C.
//   * A tiles are gathered straight from the NHWC activation (float4 along
//     the channel axis, padding taps read as zero) into LDS; B tiles come
//     from weights packed K-major [k][Co_pad4] at load time.
//   * Each wave64 owns a TM x TN grid of 16x16 accumulators and issues
//     v_mfma_f32_16x16x4f32; the next K slice is prefetched into registers
//     while the current one is multiplied.
//   * The epilogue fuses bias, activation, an SE gate on the input (applied
//     while gathering A), a (gated) residual add, a nearest-upsample add, an
//     upsample-on-write and the 2x2/stride-2 transposed-conv scatter.
#include "device_math.h"

namespace ppocr {

typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(256) void conv_gemm_kernel(ConvParams p) {
  constexpr int BK = 16;
  constexpr int TM = BM / (WM * 16);
  constexpr int TN = BN / (WN * 16);
  static_assert(WM * WN == 4, "four waves per block");
  static_assert(TM >= 1 && TN >= 1, "tile too small");
  constexpr int A_PER = BM * BK / 4 / 256;         // float4 loads of A per thread
  constexpr int B_Q = BK * BN / 4;                  // float4 count of a B tile
  constexpr int B_PER = (B_Q + 255) / 256;
  static_assert(A_PER >= 1, "BM must be a multiple of 64");

  __shared__ float As[BK][BM + 4];
  __shared__ float Bs[BK][BN + 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int HoWo = p.Ho * p.Wo;
  const int M = p.N * HoWo;
  const int K = p.kh * p.kw * p.C;
  const int cols = p.mode == 1 ? 4 * p.Co : p.Co;
  const int m0 = blockIdx.x * BM;
  const int n0 = blockIdx.y * BN;

  // Per-thread A-row geometry, fixed for the whole K loop.
  int a_img[A_PER], a_iy0[A_PER], a_ix0[A_PER];
  bool a_ok[A_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    int q = tid + i * 256;
    int m = m0 + (q >> 2);
    a_ok[i] = m < M;
    int mm = a_ok[i] ? m : 0;
    int img = mm / HoWo;
    int r = mm - img * HoWo;
    int oy = r / p.Wo;
    int ox = r - oy * p.Wo;
    a_img[i] = img;
    a_iy0[i] = oy * p.sh - p.pt;
    a_ix0[i] = ox * p.sw - p.pl;
  }

  float4 ra[A_PER];
  float4 rb[B_PER];

  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      int q = tid + i * 256;
      int k = k0 + (q & 3) * 4;
      float4 v = f4_zero();
      if (a_ok[i] && k < K) {
        int tap = k / p.C;
        int c = k - tap * p.C;
        int ky = tap / p.kw;
        int kx = tap - ky * p.kw;
        int iy = a_iy0[i] + ky;
        int ix = a_ix0[i] + kx;
        if (iy >= 0 && iy < p.H && ix >= 0 && ix < p.W) {
          v = *reinterpret_cast<const float4*>(p.in + ((size_t)(a_img[i] * p.H + iy) * p.W + ix) * p.in_ps + c);
          if (p.in_gate) {
            float4 g = *reinterpret_cast<const float4*>(p.in_gate + (size_t)a_img[i] * p.C + c);
            v.x *= g.x;
            v.y *= g.y;
            v.z *= g.z;
            v.w *= g.w;
          }
        }
      }
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      int q = tid + i * 256;
      float4 v = f4_zero();
      if (q < B_Q) {
        int kr = q / (BN / 4);
        int nq = q - kr * (BN / 4);
        int k = k0 + kr;
        int n = n0 + nq * 4;
        if (k < K && n < p.ldw) v = *reinterpret_cast<const float4*>(p.wt + (size_t)k * p.ldw + n);
      }
      rb[i] = v;
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      int q = tid + i * 256;
      int row = q >> 2;
      int kq = (q & 3) * 4;
      As[kq + 0][row] = ra[i].x;
      As[kq + 1][row] = ra[i].y;
      As[kq + 2][row] = ra[i].z;
      As[kq + 3][row] = ra[i].w;
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      int q = tid + i * 256;
      if (q < B_Q) {
        int kr = q / (BN / 4);
        int nq = q - kr * (BN / 4);
        *reinterpret_cast<float4*>(&Bs[kr][nq * 4]) = rb[i];
      }
    }
  };

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int lrow = lane & 15;
  const int lk = lane >> 4;

  load_tile(0);
  for (int k0 = 0; k0 < K; k0 += BK) {
    __syncthreads();
    store_tile();
    __syncthreads();
    if (k0 + BK < K) load_tile(k0 + BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 4) {
      float a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = As[kk + lk][wm * TM * 16 + i * 16 + lrow];
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = Bs[kk + lk][wn * TN * 16 + j * 16 + lrow];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue.  Accumulator element e of lane l in tile (i, j) is
  // row 4*(l/16) + e, column l%16 of that 16x16 tile.
  const bool need_coords = p.up != nullptr || p.rep != 1 || p.mode == 1;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int m = m0 + wm * TM * 16 + i * 16 + lk * 4 + e;
      if (m >= M) continue;
      int img = 0, oy = 0, ox = 0;
      if (need_coords) {
        img = m / HoWo;
        int r = m - img * HoWo;
        oy = r / p.Wo;
        ox = r - oy * p.Wo;
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        int col = n0 + wn * TN * 16 + j * 16 + lrow;
        if (col >= cols) continue;
        float v = acc[i][j][e];
        if (p.mode == 1) {
          int tap = col / p.Co;
          int o = col - tap * p.Co;
          if (p.bias) v = v + p.bias[o];
          v = act_apply(p.act, v);
          int y = 2 * oy + (tap >> 1);
          int x = 2 * ox + (tap & 1);
          p.out[((size_t)(img * p.out_h + y) * p.out_w + x) * p.out_ps + o] = v;
          continue;
        }
        if (p.bias) v = v + p.bias[col];
        v = act_apply(p.act, v);
        if (p.res) {
          float r = p.res[(size_t)m * p.res_ps + col];
          if (p.res_gate) r = __fmul_rn(r, p.res_gate[(size_t)(m / HoWo) * p.Co + col]);
          v = r + v;
        }
        if (p.up) {
          int uh = p.Ho / p.up_s, uw = p.Wo / p.up_s;
          v = v + p.up[((size_t)(img * uh + oy / p.up_s) * uw + ox / p.up_s) * p.up_ps + col];
        }
        if (p.rep == 1) {
          p.out[(size_t)m * p.out_ps + col] = v;
        } else {
          for (int dy = 0; dy < p.rep; ++dy)
            for (int dx = 0; dx < p.rep; ++dx)
              p.out[((size_t)(img * p.out_h + oy * p.rep + dy) * p.out_w + ox * p.rep + dx) * p.out_ps + col] = v;
        }
      }
    }
  }
}

template <int BM, int BN, int WM, int WN>
static void launch_tile(const ConvParams& p, int M, int cols, hipStream_t s) {
  dim3 grid((M + BM - 1) / BM, (cols + BN - 1) / BN);
  hipLaunchKernelGGL((conv_gemm_kernel<BM, BN, WM, WN>), grid, dim3(256), 0, s, p);
}

// Tile choice: narrow output channel counts get tall tiles so no MFMA
// column is wasted; wide layers take 128x64 when that still fills the 256
// CUs with several blocks each.
static int pick_tile(int M, int cols) {
  if (cols <= 16) return 0;
  if (cols <= 32) return 1;
  if ((long)((M + 127) / 128) * ((cols + 63) / 64) >= 1024) return 2;
  return 3;
}

const char* conv_tile_name(int M, int cols) {
  static const char* names[] = {"conv_gemm<256x16>", "conv_gemm<128x32>", "conv_gemm<128x64>", "conv_gemm<64x64>"};
  return names[pick_tile(M, cols)];
}

void launch_conv(const ConvParams& p, hipStream_t s) {
  int M = p.N * p.Ho * p.Wo;
  int cols = p.mode == 1 ? 4 * p.Co : p.Co;
  switch (pick_tile(M, cols)) {
    case 0: launch_tile<256, 16, 4, 1>(p, M, cols, s); break;
    case 1: launch_tile<128, 32, 4, 1>(p, M, cols, s); break;
    case 2: launch_tile<128, 64, 2, 2>(p, M, cols, s); break;
    default: launch_tile<64, 64, 2, 2>(p, M, cols, s); break;
  }
}

}  // namespace ppocr
