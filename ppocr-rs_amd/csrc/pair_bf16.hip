// bf16 pointwise pair of an LCNet block, fused into one launch: the
// block's channel_conv1 (1x1, C -> 2C, bias, GELU) and channel_conv2 (1x1,
// 2C -> C, bias, plus the block input as residual), with the block's SE gate
// applied to that input first (src/cpu/model.rs:509-603; the reference runs
// them as two Conv2d::forward calls and a residual add).  In a bf16 plan the
// two GEMMs otherwise run as two direct-kernel launches with the 2C-channel
// hidden tensor written to and read back from HBM (and, with a gate, a third
// pass storing x * g); here the hidden tensor never leaves registers.
//
// Layout.  The weights stay in LDS for the whole launch (one workgroup per
// CU, 8 waves): W1 [2C][C] and W2 [C][2C] are copied in once, in the order
// the MFMA reads them (one 16-byte fragment per lane, so each operand read
// is a linear, conflict-free ds_read_b128).  Each wave then streams blocks
// of 16 * MB pixel rows on its own, with no further barrier:
//   * x rows are read straight from HBM into registers as the B operand of
//     v_mfma_f32_16x16x32_bf16 (lane l: row l % 16, channels 8 (l / 16) ..
//     + 7 of each 32-channel block), multiplied by the gate and rounded to
//     bf16 where the block has one (the value the unfused plan stores);
//   * GEMM1 computes h^T = W1 x^T, 32 hidden channels at a time, with W1
//     as the A operand.  The A rows of hidden block nb are permuted (row
//     slot r holds hidden channel 32 (nb / 2) + 8 (r / 4) + 4 (nb % 2) +
//     r % 4), so that the accumulators of blocks 2j and 2j + 1 hold, in
//     lane l, hidden channels 32 j + 8 (l / 16) .. + 7 of row l % 16: after
//     bias, GELU and the bf16 rounding they are already GEMM2's B operand
//     for its k block j, with no data movement between lanes;
//   * GEMM2 accumulates out^T = W2 h^T over those k blocks with W2's rows
//     permuted the same way, so lane l ends up holding output channels
//     32 j + 8 (l / 16) .. + 7 of row l % 16: the residual (the gated,
//     rounded x) is the lane's own x fragment j, and the lane stores its
//     eight outputs as one 16-byte write.
// Both GEMMs sum over k in the same order, with the same instruction and
// the same operand positions as the direct kernel of conv_gemm.hip, and
// the epilogues round at the same points, so the result equals the unfused
// bf16 plan's bit for bit.
//
// Cost per pixel row (C = 128): 512 bytes of HBM traffic, 131 kFLOP on the
// matrix cores, and 256 GELUs on the vector ALUs, which bound the kernel.
#include <stdexcept>

#include "device_math.h"

namespace ppocr {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));

constexpr int kPairWaves = 8;

// Row of 16-row fragment block `blk` held in row slot r (see above).
__device__ __forceinline__ int frag_row(int blk, int r) {
  return 32 * (blk >> 1) + 8 * (r >> 2) + 4 * (blk & 1) + (r & 3);
}

__device__ __forceinline__ f32x4 mfma(uint4 a, uint4 b, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, a), __builtin_bit_cast(bf16x8v, b),
                                                 acc, 0, 0, 0);
}

// Eight bf16 values as floats.
__device__ __forceinline__ void unpack8(uint4 u, float (&f)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

template <int C, bool GATE, bool RES, int MB>
__global__ __launch_bounds__(64 * kPairWaves) void pair_bf16_kernel(PairBf16Params p) {
  constexpr int H = 2 * C;
  constexpr int KB = C / 32;   // GEMM1 k blocks (input channels)
  constexpr int KB2 = H / 32;  // GEMM2 k blocks (hidden channels)
  constexpr int NB = H / 16;   // hidden row blocks of GEMM1
  constexpr int CB = C / 16;   // output row blocks of GEMM2
  constexpr int ROWS = 16 * MB;
  __shared__ uint4 w1f[NB * KB * 64];
  __shared__ uint4 w2f[KB2 * CB * 64];
  __shared__ __attribute__((aligned(16))) float b1s[H];
  __shared__ __attribute__((aligned(16))) float b2s[C];

  const int tid = threadIdx.x;
  const bf16* w1 = static_cast<const bf16*>(p.w1);
  const bf16* w2 = static_cast<const bf16*>(p.w2);
  for (int q = tid; q < NB * KB * 64; q += 64 * kPairWaves) {
    const int l = q & 63, f = q >> 6, nb = f / KB, kb = f % KB;
    w1f[q] = *reinterpret_cast<const uint4*>(w1 + (size_t)frag_row(nb, l & 15) * p.ldw1 + 32 * kb + 8 * (l >> 4));
  }
  for (int q = tid; q < KB2 * CB * 64; q += 64 * kPairWaves) {
    const int l = q & 63, f = q >> 6, kb2 = f / CB, cb = f % CB;
    w2f[q] = *reinterpret_cast<const uint4*>(w2 + (size_t)frag_row(cb, l & 15) * p.ldw2 + 32 * kb2 + 8 * (l >> 4));
  }
  for (int q = tid; q < H; q += 64 * kPairWaves) b1s[q] = p.b1[q];
  for (int q = tid; q < C; q += 64 * kPairWaves) b2s[q] = p.b2[q];
  __syncthreads();

  const int lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, g = lane >> 4;
  const bf16* in = static_cast<const bf16*>(p.in);
  bf16* out = static_cast<bf16*>(p.out);
  const int nrb = (p.M + ROWS - 1) / ROWS;
  for (int rb = blockIdx.x + gridDim.x * wave; rb < nrb; rb += gridDim.x * kPairWaves) {
    // The block's x fragments (gated and rounded), zero past the last row.
    uint4 xf[MB][KB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = rb * ROWS + 16 * mb + lr;
      const bool ok = m < p.M;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
        xf[mb][kb] = ok ? *reinterpret_cast<const uint4*>(in + (size_t)m * p.in_ps + 32 * kb + 8 * g)
                        : make_uint4(0u, 0u, 0u, 0u);
      if constexpr (GATE) {
        const float* gr = p.gate + (size_t)(ok ? m / p.HW : 0) * C + 8 * g;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const float4 g0 = *reinterpret_cast<const float4*>(gr + 32 * kb);
          const float4 g1 = *reinterpret_cast<const float4*>(gr + 32 * kb + 4);
          const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
          float v[8];
          unpack8(xf[mb][kb], v);
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = mul_rn(v[i], gv[i]);
          xf[mb][kb] = pack8(v);
        }
      }
    }

    f32x4 acc[MB][CB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) acc[mb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll 1
    for (int j = 0; j < KB2; ++j) {
      // GEMM1 for hidden channels 32 j .. 32 j + 31.
      f32x4 h0[MB], h1[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) h0[mb] = h1[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const uint4 wa = w1f[((2 * j) * KB + kb) * 64 + lane];
        const uint4 wb = w1f[((2 * j + 1) * KB + kb) * 64 + lane];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          h0[mb] = mfma(wa, xf[mb][kb], h0[mb]);
          h1[mb] = mfma(wb, xf[mb][kb], h1[mb]);
        }
      }
      // Bias, GELU, bf16: GEMM2's operand for its k block j.
      const float4 bl = *reinterpret_cast<const float4*>(b1s + 32 * j + 8 * g);
      const float4 bh = *reinterpret_cast<const float4*>(b1s + 32 * j + 8 * g + 4);
      uint4 hf[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const float v[8] = {gelu_as(h0[mb][0] + bl.x), gelu_as(h0[mb][1] + bl.y), gelu_as(h0[mb][2] + bl.z),
                            gelu_as(h0[mb][3] + bl.w), gelu_as(h1[mb][0] + bh.x), gelu_as(h1[mb][1] + bh.y),
                            gelu_as(h1[mb][2] + bh.z), gelu_as(h1[mb][3] + bh.w)};
        hf[mb] = pack8(v);
      }
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const uint4 w = w2f[(j * CB + cb) * 64 + lane];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb][cb] = mfma(w, hf[mb], acc[mb][cb]);
      }
    }

    // Bias, residual, bf16: output channels 32 j + 8 g .. + 7 of the lane's row.
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const float4 bl = *reinterpret_cast<const float4*>(b2s + 32 * j + 8 * g);
      const float4 bh = *reinterpret_cast<const float4*>(b2s + 32 * j + 8 * g + 4);
      const float bv[8] = {bl.x, bl.y, bl.z, bl.w, bh.x, bh.y, bh.z, bh.w};
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int m = rb * ROWS + 16 * mb + lr;
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = acc[mb][2 * j][e] + bv[e];
          v[4 + e] = acc[mb][2 * j + 1][e] + bv[4 + e];
        }
        if constexpr (RES) {
          float r[8];
          unpack8(xf[mb][j], r);
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = r[i] + v[i];
        }
        if (m < p.M) *reinterpret_cast<uint4*>(out + (size_t)m * p.out_ps + 32 * j + 8 * g) = pack8(v);
      }
    }
  }
}

// Rows per wave block: 32 where that still gives every wave of the grid a
// block, else 16.
int pair_rows(int M) {
  const long slots = (long)device_cus() * kPairWaves;
  return (M + 31) / 32 >= slots ? 32 : 16;
}

template <int C, int MB>
void launch_c(const PairBf16Params& p, hipStream_t s) {
  const int nrb = (p.M + 16 * MB - 1) / (16 * MB);
  const dim3 grid((unsigned)std::max(1, std::min(device_cus(), nrb)));
  const dim3 block(64 * kPairWaves);
  if (p.gate) {
    if (p.residual)
      hipLaunchKernelGGL((pair_bf16_kernel<C, true, true, MB>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((pair_bf16_kernel<C, true, false, MB>), grid, block, 0, s, p);
  } else {
    if (p.residual)
      hipLaunchKernelGGL((pair_bf16_kernel<C, false, true, MB>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((pair_bf16_kernel<C, false, false, MB>), grid, block, 0, s, p);
  }
}

template <int C>
void launch_rows(const PairBf16Params& p, hipStream_t s) {
  if (pair_rows(p.M) == 32)
    launch_c<C, 2>(p, s);
  else
    launch_c<C, 1>(p, s);
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

}  // namespace

bool pair_bf16_supported(int C, int H2, int Co) { return (C == 64 || C == 96 || C == 128) && H2 == 2 * C && Co == C; }

std::string pair_bf16_kernel_name(const PairBf16Params& p) {
  return "pair_bf16<" + std::to_string(p.C) + "," + std::to_string(pair_rows(p.M)) + (p.gate ? ",gate" : "") +
         (p.residual ? ",res" : "") + ">";
}

void launch_pair_bf16(const PairBf16Params& p, hipStream_t s) {
  if (!pair_bf16_supported(p.C, 2 * p.C, p.C) || p.M < 0 || (p.gate && p.HW <= 0))
    throw std::runtime_error("pair_bf16: unsupported shape");
  if (p.in_ps % 8 || p.out_ps % 8 || p.ldw1 % 8 || p.ldw2 % 8 || p.in_ps < p.C || p.out_ps < p.C ||
      p.ldw1 < p.C || p.ldw2 < 2 * p.C || !aligned16(p.in) || !aligned16(p.out) || !aligned16(p.w1) ||
      !aligned16(p.w2) || (p.gate && !aligned16(p.gate)))
    throw std::runtime_error("pair_bf16: rows and weights must be 16-byte aligned");
  if (p.M == 0) return;
  switch (p.C) {
    case 64: launch_rows<64>(p, s); break;
    case 96: launch_rows<96>(p, s); break;
    default: launch_rows<128>(p, s); break;
  }
}

}  // namespace ppocr
