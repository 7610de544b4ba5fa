// Implicit-GEMM convolution on the CDNA4 fp32 matrix cores.
//
// Replaces the reference's WGSL `conv`, `conv_medium_linear`,
// `conv_single_row`, `conv_spatial_m32`, `conv_2x2_direct`,
// `conv_3x3_stride2_direct`, `conv_3x3_direct` (src/gpu/shaders/*.wgsl;
// kernel selection src/gpu/runtime.rs:699-949) with one tiled kernel:
//   * M = output pixels (NHWC rows), N = output channels, K = kh*kw*C.
//   * A tiles are gathered straight from the NHWC activation (float4 along
//     the channel axis, padding taps read as zero); B tiles come from weights
//     packed [Co][K] at load time.  Both are stored k-contiguous in LDS, so
//     each lane fetches the operands of four consecutive MFMA k-steps with
//     one 16-byte LDS read.
//   * Each wave64 owns a TM x TN grid of 16x16 accumulators and issues
//     v_mfma_f32_16x16x4f32.  LDS is double-buffered: the next K slice is
//     fetched into registers during the MFMAs and written to the other
//     buffer, one barrier per slice.
//   * The epilogue stages the tile through LDS and finishes it with 16-byte
//     row-contiguous accesses: bias, activation, SE gate on the input
//     (applied while gathering A), a (gated) residual add, a
//     nearest-upsample add and an upsample-on-write.
#include "device_math.h"

namespace ppocr {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 f4_add(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(256) void conv_gemm_kernel(ConvParams p) {
  constexpr int BK = 16, KQ = BK / 4, LDA = BK + 4;
  constexpr int TM = BM / (WM * 16);
  constexpr int TN = BN / (WN * 16);
  static_assert(WM * WN == 4, "four waves per block");
  static_assert(TM >= 1 && TN >= 1, "tile too small");
  constexpr int A_PER = BM * KQ / 256;  // float4 loads of A per thread
  constexpr int B_Q = BN * KQ;          // float4 count of a B tile
  constexpr int B_PER = (B_Q + 255) / 256;
  static_assert(A_PER >= 1, "BM must be a multiple of 64");
  constexpr int STAGE = (BM + BN) * LDA;
  constexpr int LDE = BN + 4;
  constexpr int SMEM = 2 * STAGE > BM * LDE ? 2 * STAGE : BM * LDE;
  __shared__ __attribute__((aligned(16))) float smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int HoWo = p.Ho * p.Wo;
  const int M = p.N * HoWo;
  const int K = p.kh * p.kw * p.C;
  const int m0 = blockIdx.x * BM;
  const int n0 = blockIdx.y * BN;
  const int kq = tid % KQ;  // this lane's k-quad in every A and B load

  // Per-thread A-row geometry, fixed for the whole K loop.
  int a_img[A_PER], a_iy0[A_PER], a_ix0[A_PER];
  bool a_ok[A_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    int m = m0 + (tid + i * 256) / KQ;
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
    const int k = k0 + kq * 4;
    const bool kin = k < K;
    const int tap = k / p.C;
    const int c = k - tap * p.C;
    const int ky = tap / p.kw;
    const int kx = tap - ky * p.kw;
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      float4 v = f4_zero();
      int iy = a_iy0[i] + ky;
      int ix = a_ix0[i] + kx;
      if (kin && a_ok[i] && iy >= 0 && iy < p.H && ix >= 0 && ix < p.W) {
        v = *reinterpret_cast<const float4*>(p.in + ((size_t)(a_img[i] * p.H + iy) * p.W + ix) * p.in_ps + c);
        if (p.in_gate) {
          float4 g = *reinterpret_cast<const float4*>(p.in_gate + (size_t)a_img[i] * p.C + c);
          v.x *= g.x;
          v.y *= g.y;
          v.z *= g.z;
          v.w *= g.w;
        }
      }
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      int q = tid + i * 256;
      int n = n0 + q / KQ;
      float4 v = f4_zero();
      if (q < B_Q && kin && n < p.Co) v = *reinterpret_cast<const float4*>(p.wt + (size_t)n * p.ldw + k);
      rb[i] = v;
    }
  };

  auto store_tile = [&](int buf) {
    float* As = smem + buf * STAGE;
    float* Bs = As + BM * LDA;
#pragma unroll
    for (int i = 0; i < A_PER; ++i)
      *reinterpret_cast<float4*>(As + ((tid + i * 256) / KQ) * LDA + kq * 4) = ra[i];
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      int q = tid + i * 256;
      if (q < B_Q) *reinterpret_cast<float4*>(Bs + (q / KQ) * LDA + kq * 4) = rb[i];
    }
  };

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // MFMA operand mapping: lane l supplies A[m = l%16][k] and B[k][n = l%16];
  // over four MFMA steps lane group g = l/16 covers k = 4g .. 4g+3, read as
  // one float4 (the k order within a slice is permuted identically for A and
  // B, so the products pair up unchanged).
  const int lrow = lane & 15;
  const int g = lane >> 4;
  const int nk = (K + BK - 1) / BK;

  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int s = 0; s < nk; ++s) {
    const int buf = s & 1;
    if (s + 1 < nk) load_tile((s + 1) * BK);
    const float* As = smem + buf * STAGE;
    const float* Bs = As + BM * LDA;
    float4 a[TM], b[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
      a[i] = *reinterpret_cast<const float4*>(As + (wm * TM * 16 + i * 16 + lrow) * LDA + g * 4);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      b[j] = *reinterpret_cast<const float4*>(Bs + (wn * TN * 16 + j * 16 + lrow) * LDA + g * 4);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
    if (s + 1 < nk) store_tile(buf ^ 1);
    __syncthreads();
  }

  // Stage the tile in LDS as [m][n].  Accumulator element e of lane l in
  // tile (i, j) is row 4*(l/16) + e, column l%16 of that 16x16 tile.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        smem[(wm * TM * 16 + i * 16 + g * 4 + e) * LDE + wn * TN * 16 + j * 16 + lrow] = acc[i][j][e];
  __syncthreads();

  const bool vec_out = (p.out_ps & 3) == 0 && (p.Co & 3) == 0;
  const bool need_coords = p.up != nullptr || p.rep != 1;
  constexpr int NQ = BN / 4;
  for (int q = tid; q < BM * NQ; q += 256) {
    const int row = q / NQ;
    const int cq = q - row * NQ;
    const int m = m0 + row;
    const int col = n0 + cq * 4;
    if (m >= M || col >= p.Co) continue;
    float4 v = *reinterpret_cast<const float4*>(smem + row * LDE + cq * 4);
    int img = m / HoWo, oy = 0, ox = 0;
    if (need_coords) {
      int r = m - img * HoWo;
      oy = r / p.Wo;
      ox = r - oy * p.Wo;
    }
    if (vec_out) {
      if (p.bias) v = f4_add(v, *reinterpret_cast<const float4*>(p.bias + col));
      v.x = act_apply(p.act, v.x);
      v.y = act_apply(p.act, v.y);
      v.z = act_apply(p.act, v.z);
      v.w = act_apply(p.act, v.w);
      if (p.res) {
        float4 r = *reinterpret_cast<const float4*>(p.res + (size_t)m * p.res_ps + col);
        if (p.res_gate) {
          float4 gt = *reinterpret_cast<const float4*>(p.res_gate + (size_t)img * p.Co + col);
          r = make_float4(__fmul_rn(r.x, gt.x), __fmul_rn(r.y, gt.y), __fmul_rn(r.z, gt.z), __fmul_rn(r.w, gt.w));
        }
        v = f4_add(r, v);
      }
      if (p.up) {
        int uh = p.Ho / p.up_s, uw = p.Wo / p.up_s;
        v = f4_add(v, *reinterpret_cast<const float4*>(
                          p.up + ((size_t)(img * uh + oy / p.up_s) * uw + ox / p.up_s) * p.up_ps + col));
      }
      if (p.rep == 1) {
        *reinterpret_cast<float4*>(p.out + (size_t)m * p.out_ps + col) = v;
      } else {
        for (int dy = 0; dy < p.rep; ++dy)
          for (int dx = 0; dx < p.rep; ++dx)
            *reinterpret_cast<float4*>(
                p.out + ((size_t)(img * p.out_h + oy * p.rep + dy) * p.out_w + ox * p.rep + dx) * p.out_ps + col) = v;
      }
    } else {
      // Channel counts that are not a multiple of 4 (the recognizer
      // classifiers, 6906 and 18710) go element by element; they carry no
      // residual, gate or upsample terms.
      const float vv[4] = {v.x, v.y, v.z, v.w};
      for (int e = 0; e < 4 && col + e < p.Co; ++e) {
        float t = vv[e];
        if (p.bias) t = t + p.bias[col + e];
        p.out[(size_t)m * p.out_ps + col + e] = act_apply(p.act, t);
      }
    }
  }
}

template <int BM, int BN, int WM, int WN>
static void launch_tile(const ConvParams& p, int M, hipStream_t s) {
  dim3 grid((M + BM - 1) / BM, (p.Co + BN - 1) / BN);
  hipLaunchKernelGGL((conv_gemm_kernel<BM, BN, WM, WN>), grid, dim3(256), 0, s, p);
}

// Tile choice: narrow output channel counts get tall tiles so no MFMA
// column is wasted; wide layers take 128x64 when that still gives every CU
// several blocks.
static int pick_tile(int M, int cols) {
  if (cols <= 16) return 0;
  if (cols <= 32) return 1;
  if ((long)((M + 127) / 128) * ((cols + 63) / 64) >= 2048) return 2;
  return 3;
}

const char* conv_tile_name(int M, int cols) {
  static const char* names[] = {"conv_gemm<256x16>", "conv_gemm<128x32>", "conv_gemm<128x64>", "conv_gemm<64x64>"};
  return names[pick_tile(M, cols)];
}

void launch_conv(const ConvParams& p, hipStream_t s) {
  int M = p.N * p.Ho * p.Wo;
  switch (pick_tile(M, p.Co)) {
    case 0: launch_tile<256, 16, 4, 1>(p, M, s); break;
    case 1: launch_tile<128, 32, 4, 1>(p, M, s); break;
    case 2: launch_tile<128, 64, 2, 2>(p, M, s); break;
    default: launch_tile<64, 64, 2, 2>(p, M, s); break;
  }
}

}  // namespace ppocr
