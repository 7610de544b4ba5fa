// Implicit-GEMM convolution on the CDNA4 matrix cores, fp32 or bf16 storage.
//
// Replaces the reference's WGSL `conv`, `conv_medium_linear`,
// `conv_single_row`, `conv_spatial_m32`, `conv_2x2_direct`,
// `conv_3x3_stride2_direct`, `conv_3x3_direct` (src/gpu/shaders/*.wgsl;
// kernel selection src/gpu/runtime.rs:699-949) with one tiled kernel:
//   * M = output pixels (NHWC rows), N = output channels, K = kh*kw*C.
//   * A tiles are gathered straight from the NHWC activation (four channels
//     per load, padding taps read as zero); B tiles come from weights packed
//     [Co][K] at load time.  Both are stored k-contiguous in LDS with 80-byte
//     rows, so each lane fetches its MFMA operands for one K slice with one
//     conflict-free 16-byte LDS read per 16x16 tile.
//   * fp32: v_mfma_f32_16x16x4f32, four per tile per 16-deep K slice.
//     bf16: v_mfma_f32_16x16x32_bf16, one per tile per 32-deep K slice, fp32
//     accumulation.
//   * Each wave64 owns a TM x TN grid of 16x16 accumulators.
//   * Most layers run conv_gemm_direct_kernel: operand rows are loaded
//     straight into LDS (buffer_load_dwordx4 ... lds) through a 3- or
//     4-stage pipeline; fp32 1x1 layers with an SE input gate multiply the A
//     fragments by gate rows staged in LDS.  The other gated layers (the gate
//     multiplies A while it is gathered) and bf16 layers whose channel count
//     is not a multiple of 8 run conv_gemm_kernel: the next K slice is
//     fetched into registers during the MFMAs and written to the other of
//     two LDS buffers.
//   * The epilogue stages the fp32 tile through LDS and finishes it with
//     row-contiguous vector accesses: bias, activation, SE gate on the input
//     (applied while gathering A), a (gated) residual add, a
//     nearest-upsample add and an upsample-on-write.
#include <type_traits>

#include <atomic>
#include <stdexcept>

#include "device_math.h"

namespace ppocr {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <typename T>
struct GemmTraits;
template <>
struct GemmTraits<float> {
  static constexpr int BK = 16;  // K slice: 16 fp32 = 64 B per row
};
template <>
struct GemmTraits<bf16> {
  static constexpr int BK = 32;  // K slice: 32 bf16 = 64 B per row
};

// A global-load vector of VE consecutive k values: 16 bytes (fp32 x4,
// bf16 x8), or 8 bytes (bf16 x4) for layers whose channel count is not a
// multiple of 8.
template <typename T, int VE>
struct VecT;
template <>
struct VecT<float, 4> {
  using type = float4;
};
template <>
struct VecT<bf16, 8> {
  using type = uint4;
};
template <>
struct VecT<bf16, 4> {
  using type = uint2;
};

__device__ __forceinline__ float4 f4_add(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__device__ __forceinline__ uint32_t gate_pair(uint32_t v, float g0, float g1) {
  return pack_bf16x2(bf16_bits_to_f32(v & 0xFFFFu) * g0, bf16_bits_to_f32(v >> 16) * g1);
}

// v * g elementwise (the SE gate applied while gathering A); g points at the
// VE gate values of these channels.
__device__ __forceinline__ float4 gate_vec(float4 v, const float* g) {
  return f4_mul(v, *reinterpret_cast<const float4*>(g));
}
__device__ __forceinline__ uint2 gate_vec(uint2 v, const float* g) {
  const float4 a = *reinterpret_cast<const float4*>(g);
  return make_uint2(gate_pair(v.x, a.x, a.y), gate_pair(v.y, a.z, a.w));
}
__device__ __forceinline__ uint4 gate_vec(uint4 v, const float* g) {
  const float4 a = *reinterpret_cast<const float4*>(g), b = *reinterpret_cast<const float4*>(g + 4);
  return make_uint4(gate_pair(v.x, a.x, a.y), gate_pair(v.y, a.z, a.w), gate_pair(v.z, b.x, b.y),
                    gate_pair(v.w, b.z, b.w));
}

template <typename T, int BM, int BN, int WM, int WN, typename RowPtr>
__device__ __forceinline__ void finish_tile(const ConvParams& p, const floatx4 (&acc)[BM / (WM * 16)][BN / (WN * 16)],
                                            RowPtr row_ptr, int m0, int n0, int M, int n_tiles);

// PW: 1x1 convolution with stride 1 and no padding, where an output pixel
// reads exactly its own input pixel and A rows are plain strided rows.
// VE: k values per global load (see VecT).
template <typename T, int BM, int BN, int WM, int WN, bool PW, int VE>
__global__ __launch_bounds__(256) void conv_gemm_kernel(ConvParams p) {
  using Vec = typename VecT<T, VE>::type;
  constexpr int BK = GemmTraits<T>::BK;
  constexpr int KV = BK / VE;                // vectors per row of a K slice
  constexpr int RPP = 256 / KV;              // tile rows loaded per pass of the block
  constexpr int PADE = 16 / sizeof(T);       // 16 B of padding per LDS row
  constexpr int LDA = BK + PADE;             // 80-byte rows
  constexpr int OPE = 16 / sizeof(T);        // elements per 16-byte operand read
  constexpr int TM = BM / (WM * 16);
  constexpr int TN = BN / (WN * 16);
  static_assert(WM * WN == 4, "four waves per block");
  static_assert(TM >= 1 && TN >= 1, "tile too small");
  static_assert(BM % RPP == 0, "A tile must split evenly over the block");
  constexpr int A_PER = BM / RPP;
  constexpr int B_PER = (BN + RPP - 1) / RPP;
  constexpr int STAGE = (BM + BN) * LDA;     // elements of T
  constexpr int LDE = BN + 4;                // fp32 epilogue staging
  constexpr int SMEM_BYTES = 2 * STAGE * (int)sizeof(T) > BM * LDE * 4 ? 2 * STAGE * (int)sizeof(T) : BM * LDE * 4;
  __shared__ __attribute__((aligned(16))) char smem_raw[SMEM_BYTES];
  T* smem = reinterpret_cast<T*>(smem_raw);

  const T* in = static_cast<const T*>(p.in);
  const T* wt = static_cast<const T*>(p.wt);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int HoWo = p.Ho * p.Wo;
  const int M = p.N * HoWo;
  const int K = p.kh * p.kw * p.C;

  // XCD-aware tile order.  Workgroups are dealt round-robin to the 8 XCDs,
  // each with its own L2.  Workgroup w runs on XCD w % 8 and is given tile
  // (w % 8) * per_xcd + w / 8 of the (M-tile, N-tile) list in M-major
  // order, so every XCD walks a contiguous run of M tiles with all their N
  // tiles back to back: an activation tile is fetched into one L2 once and
  // reused by every N tile instead of being re-fetched per N tile.
  const int n_tiles = (p.Co + BN - 1) / BN;
  const int m_tiles = (M + BM - 1) / BM;
  const int per_xcd = gridDim.x / 8;
  const int t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (t >= m_tiles * n_tiles) return;
  const int m0 = (t / n_tiles) * BM;
  const int n0 = (t % n_tiles) * BN;
  const int kv = tid % KV;    // this lane's vector within a row of the K slice
  const int rrow = tid / KV;  // this lane's first tile row; then every RPP rows

  // A rows.  PW: a row is the input pixel itself.  Otherwise: image and the
  // top-left input coordinate of the output pixel's window.
  const T* a_ptr[A_PER];
  int a_img[A_PER], a_iy0[A_PER], a_ix0[A_PER];
  bool a_ok[A_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int m = m0 + rrow + i * RPP;
    a_ok[i] = m < M;
    const int mm = a_ok[i] ? m : 0;
    const int img = mm / HoWo;
    a_img[i] = img;
    if constexpr (PW) {
      a_ptr[i] = in + (size_t)mm * p.in_ps;
      a_iy0[i] = a_ix0[i] = 0;
    } else {
      const int r = mm - img * HoWo;
      const int oy = r / p.Wo;
      const int ox = r - oy * p.Wo;
      a_ptr[i] = in + (size_t)img * p.H * p.W * p.in_ps;
      a_iy0[i] = oy * p.sh - p.pt;
      a_ix0[i] = ox * p.sw - p.pl;
    }
  }
  bool b_ok[B_PER];
  const T* b_ptr[B_PER];
#pragma unroll
  for (int i = 0; i < B_PER; ++i) {
    const int r = rrow + i * RPP;
    const int n = n0 + r;
    b_ok[i] = r < BN && n < p.Co;
    b_ptr[i] = wt + (size_t)(b_ok[i] ? n : 0) * p.ldw;
  }

  // K slices of this workgroup: all of them, or its split's share.
  const int nk_all = (K + BK - 1) / BK;
  const int s_begin = (int)((long)blockIdx.y * nk_all / gridDim.y);
  const int nk = (int)((long)(blockIdx.y + 1) * nk_all / gridDim.y) - s_begin;
  const int kbase = s_begin * BK;

  // Decomposition of this lane's k = k0 + kv*VE into (ky, kx, c), kept up to
  // date as the K slices advance (one division at the start, none in the
  // loop).  A vector never straddles a tap: C is a multiple of VE.
  int kc = kbase + kv * VE, kx = 0, ky = 0;
  if constexpr (!PW) {
    const int tap = kc / p.C;
    kc -= tap * p.C;
    ky = tap / p.kw;
    kx = tap - ky * p.kw;
  }

  Vec ra[A_PER], rb[B_PER];

  // Loads the K slice starting at k0 (called for k0 = kbase, kbase + BK,
  // ... in order) into registers.
  auto load_tile = [&](Vec(&ra)[A_PER], Vec(&rb)[B_PER], int k0) {
    const int k = k0 + kv * VE;
    const bool kin = k < K;
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      Vec v{};
      if constexpr (PW) {
        if (kin && a_ok[i]) {
          v = *reinterpret_cast<const Vec*>(a_ptr[i] + k);
          if (p.in_gate) v = gate_vec(v, p.in_gate + (size_t)a_img[i] * p.C + k);
        }
      } else {
        const int iy = a_iy0[i] + ky;
        const int ix = a_ix0[i] + kx;
        if (kin && a_ok[i] && iy >= 0 && iy < p.H && ix >= 0 && ix < p.W) {
          v = *reinterpret_cast<const Vec*>(a_ptr[i] + ((size_t)iy * p.W + ix) * p.in_ps + kc);
          if (p.in_gate) v = gate_vec(v, p.in_gate + (size_t)a_img[i] * p.C + kc);
        }
      }
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      Vec v{};
      if (kin && b_ok[i]) v = *reinterpret_cast<const Vec*>(b_ptr[i] + k);
      rb[i] = v;
    }
    if constexpr (!PW) {
      kc += BK;
      while (kc >= p.C) {
        kc -= p.C;
        if (++kx == p.kw) {
          kx = 0;
          ++ky;
        }
      }
    }
  };

  auto store_tile = [&](const Vec(&ra)[A_PER], const Vec(&rb)[B_PER], int buf) {
    T* As = smem + buf * STAGE;
    T* Bs = As + BM * LDA;
#pragma unroll
    for (int i = 0; i < A_PER; ++i) *reinterpret_cast<Vec*>(As + (rrow + i * RPP) * LDA + kv * VE) = ra[i];
#pragma unroll
    for (int i = 0; i < B_PER; ++i)
      if (rrow + i * RPP < BN) *reinterpret_cast<Vec*>(Bs + (rrow + i * RPP) * LDA + kv * VE) = rb[i];
  };

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // MFMA operand mapping: lane l supplies A[m = l%16][k] and B[k][n = l%16]
  // for the k values of its lane group g = l/16 (fp32: k = 4g..4g+3 over
  // four MFMAs; bf16: k = 8g..8g+7 in one MFMA).  The k order inside a slice
  // is the same for A and B, so the products pair up unchanged.
  const int lrow = lane & 15;
  const int g = lane >> 4;

  auto compute = [&](int buf) {
    const T* As = smem + buf * STAGE;
    const T* Bs = As + BM * LDA;
    if constexpr (sizeof(T) == 4) {
      float4 a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *reinterpret_cast<const float4*>(As + (wm * TM * 16 + i * 16 + lrow) * LDA + g * OPE);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        b[j] = *reinterpret_cast<const float4*>(Bs + (wn * TN * 16 + j * 16 + lrow) * LDA + g * OPE);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
    } else {
      bf16x8 a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *reinterpret_cast<const bf16x8*>(As + (wm * TM * 16 + i * 16 + lrow) * LDA + g * OPE);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        b[j] = *reinterpret_cast<const bf16x8*>(Bs + (wn * TN * 16 + j * 16 + lrow) * LDA + g * OPE);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };

  // Double-buffered LDS: the next slice's loads are in flight in registers
  // while this slice is multiplied, then stored to the other buffer.
  load_tile(ra, rb, kbase);
  store_tile(ra, rb, 0);
  __syncthreads();
  for (int s = 0; s < nk; ++s) {
    if (s + 1 < nk) load_tile(ra, rb, kbase + (s + 1) * BK);
    compute(s & 1);
    if (s + 1 < nk) store_tile(ra, rb, (s + 1) & 1);
    __syncthreads();
  }

  float* stage = reinterpret_cast<float*>(smem_raw);
  finish_tile<T, BM, BN, WM, WN>(
      p, acc, [=](int row) { return stage + row * LDE; }, m0, n0, M, n_tiles, nullptr);
}

// Epilogue of four consecutive output columns col..col+3 of row m (Co and
// out_ps multiples of 4), in two phases so that a tile's loads are all in
// flight before its first store (the compiler cannot move a load above a
// store that may alias it, and each load would otherwise cost a full memory
// latency): epilogue_load reads the memory terms, the (gated) residual r and
// the upsample-add source u; epilogue_store adds the bias b, applies the
// activation, adds r then u, and stores (plain, fp32, or upsample-on-write).
// img, oy, ox: the row's image and output coordinates, read only by the
// terms that use them.
struct EpiTerms {
  float4 r, u;
};

template <typename T>
__device__ __forceinline__ EpiTerms epilogue_load(const ConvParams& p, int m, int col, int img, int oy, int ox) {
  EpiTerms t{};
  if (p.res) {
    t.r = ld4<T>(static_cast<const T*>(p.res) + (size_t)m * p.res_ps + col);
    if (p.res_gate) {
      const float4 gt = *reinterpret_cast<const float4*>(p.res_gate + (size_t)img * p.Co + col);
      t.r = make_float4(mul_rn(t.r.x, gt.x), mul_rn(t.r.y, gt.y), mul_rn(t.r.z, gt.z), mul_rn(t.r.w, gt.w));
    }
  }
  if (p.up) {
    const int uh = p.Ho / p.up_s, uw = p.Wo / p.up_s;
    t.u = ld4<T>(static_cast<const T*>(p.up) + ((size_t)(img * uh + oy / p.up_s) * uw + ox / p.up_s) * p.up_ps +
                 col);
  }
  return t;
}

// Bias of columns col..col+3 (zero without a bias or past Co).
__device__ __forceinline__ float4 bias4(const ConvParams& p, int col) {
  return p.bias && col + 3 < p.Co ? *reinterpret_cast<const float4*>(p.bias + col) : float4{0.f, 0.f, 0.f, 0.f};
}

// Returns the value stored (rounded to the storage type).
template <typename T>
__device__ __forceinline__ float4 epilogue_store(const ConvParams& p, float4 v, float4 b, const EpiTerms& t, int m,
                                                 int col, int img, int oy, int ox) {
  if (p.bias) v = f4_add(v, b);
  v.x = act_apply(p.act, v.x);
  v.y = act_apply(p.act, v.y);
  v.z = act_apply(p.act, v.z);
  v.w = act_apply(p.act, v.w);
  if (p.res) v = f4_add(t.r, v);
  if (p.up) v = f4_add(v, t.u);
  if (p.out_f32) {
    *reinterpret_cast<float4*>(static_cast<float*>(p.out) + (size_t)m * p.out_ps + col) = v;
    return v;
  } else if (p.rep == 1) {
    st4<T>(static_cast<T*>(p.out) + (size_t)m * p.out_ps + col, v);
  } else if (p.rep_split) {
    T* row = static_cast<T*>(p.out) + ((size_t)(img * p.out_h + oy * p.rep + (int)blockIdx.z) * p.out_w + ox * p.rep) * p.out_ps + col;
    for (int dx = 0; dx < p.rep; ++dx) st4<T>(row + (size_t)dx * p.out_ps, v);
  } else {
    for (int dy = 0; dy < p.rep; ++dy)
      for (int dx = 0; dx < p.rep; ++dx)
        st4<T>(static_cast<T*>(p.out) +
                   ((size_t)(img * p.out_h + oy * p.rep + dy) * p.out_w + ox * p.rep + dx) * p.out_ps + col,
               v);
  }
  return round4<T>(v);
}

template <typename T, int BM, int BN, typename RowPtr>
__device__ __forceinline__ void finish_staged(const ConvParams& p, RowPtr row_ptr, int m0, int n0, int M,
                                              int n_tiles, const float4* bias_pre);

// Stages the fp32 accumulator tile in LDS as [m][n] (row_ptr(r): LDS
// address of staged row r, BN + 4 floats) and finishes it: with split K
// (p.splits > 1) the tile goes to this split's plane of the workspace as is,
// otherwise through the epilogue.  Caller has passed a barrier after its
// last read of the LDS operand buffers.  bias_pre: null, or the bias of this
// thread's staged-epilogue columns (staged_col) loaded ahead.
template <typename T, int BM, int BN, int WM, int WN, typename RowPtr>
__device__ __forceinline__ void finish_tile(const ConvParams& p, const floatx4 (&acc)[BM / (WM * 16)][BN / (WN * 16)],
                                            RowPtr row_ptr, int m0, int n0, int M, int n_tiles,
                                            const float4* bias_pre) {
  constexpr int TM = BM / (WM * 16);
  constexpr int TN = BN / (WN * 16);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lrow = lane & 15;
  const int g = lane >> 4;

  // Accumulator element e of lane l in tile (i, j) is row 4*(l/16) + e,
  // column l%16 of that 16x16 tile.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        row_ptr(wm * TM * 16 + i * 16 + g * 4 + e)[wn * TN * 16 + j * 16 + lrow] = acc[i][j][e];
  __syncthreads();
  if (p.splits > 1) {
    // Co is a multiple of 4 for split layers: whole float4 rows.
    float* ws = p.split_ws + (size_t)blockIdx.y * M * p.Co;
    constexpr int NQ = BN / 4;
    for (int q = tid; q < BM * NQ; q += 256) {
      const int row = q / NQ;
      const int col = n0 + (q - row * NQ) * 4;
      const int m = m0 + row;
      if (m < M && col < p.Co)
        *reinterpret_cast<float4*>(ws + (size_t)m * p.Co + col) =
            *reinterpret_cast<const float4*>(row_ptr(row) + (col - n0));
    }
    return;
  }
  finish_staged<T, BM, BN>(p, row_ptr, m0, n0, M, n_tiles, bias_pre);
}

// First column of a thread's float4 groups in the staged epilogue: 256
// threads walk the tile's BN / 4 groups per row, and BN / 4 divides 256, so
// a thread keeps the same column group in every row it finishes.
template <int BN>
__device__ __forceinline__ int staged_col(int n0) {
  static_assert(256 % (BN / 4) == 0, "fixed column group per thread");
  return n0 + (threadIdx.x % (BN / 4)) * 4;
}

// Epilogue of a tile staged in LDS: the greedy-CTC row reduction, or bias,
// activation, (gated) residual, upsample-add and the store (plain, fp32, or
// upsample-on-write).
template <typename T, int BM, int BN, typename RowPtr>
__device__ __forceinline__ void finish_staged(const ConvParams& p, RowPtr row_ptr, int m0, int n0, int M,
                                              int n_tiles, const float4* bias_pre) {
  const int tid = threadIdx.x;
  const int HoWo = p.Ho * p.Wo;

  // DB head tail.  Pass 1: u = ReLU(staged + bias) in place.  Pass 2: for
  // each (row, tap) of the tile, f[q] = sum_o u[o] * wf[o][q] over the
  // tap's db_ch hidden channels; tpi lanes share an item, each summing a
  // contiguous quarter or half of o, combined with xor shuffles; then
  // sigmoid(f + bf) into the 2x2 output block of the tap
  // (src/cpu/model.rs:1516-1520).
  if (p.db_ch) {
    const int ch = p.db_ch;
    for (int q = tid; q < BM * BN; q += 256) {
      const int row = q / BN, c = q - row * BN;
      float* r = row_ptr(row);
      r[c] = fmaxf(r[c] + p.bias[n0 + c], 0.0f);
    }
    __syncthreads();
    const int taps = BN / ch;
    const int items = BM * taps;
    const int tpi = items >= 256 ? 1 : 256 / items;  // 1, 2 or 4 (ch <= 64, BM >= 64)
    const int per = ch / tpi;
    const int OW = 4 * p.Wo;
    float* map = static_cast<float*>(p.out);
    for (int base = 0; base < items * tpi; base += 256) {
      const int it = base + tid;
      const int item = it / tpi, sub = it - item * tpi;
      const int row = item / taps, tl = item - row * taps;
      const float* u = row_ptr(min(row, BM - 1)) + tl * ch + sub * per;
      const float* w = p.db_wf + sub * per * 4;
      float f0 = 0.f, f1 = 0.f, f2 = 0.f, f3 = 0.f;
      for (int o = 0; o < per; ++o) {
        const float4 wq = *reinterpret_cast<const float4*>(w + o * 4);
        const float v = u[o];
        f0 = fmaf(v, wq.x, f0);
        f1 = fmaf(v, wq.y, f1);
        f2 = fmaf(v, wq.z, f2);
        f3 = fmaf(v, wq.w, f3);
      }
      for (int s = 1; s < tpi; s <<= 1) {
        f0 += __shfl_xor(f0, s);
        f1 += __shfl_xor(f1, s);
        f2 += __shfl_xor(f2, s);
        f3 += __shfl_xor(f3, s);
      }
      const int m = m0 + row;
      if (item >= items || m >= M) continue;
      const int img = m / HoWo, r = m - img * HoWo;
      const int y = r / p.Wo, x = r - y * p.Wo;
      const int tap = n0 / ch + tl;
      float* top = map + ((size_t)img * 4 * p.Ho + 4 * y + 2 * (tap >> 1)) * OW + 4 * x + 2 * (tap & 1);
      const float s0 = act_apply(ACT_SIGMOID, f0 + p.db_bf), s1 = act_apply(ACT_SIGMOID, f1 + p.db_bf);
      const float s2 = act_apply(ACT_SIGMOID, f2 + p.db_bf), s3 = act_apply(ACT_SIGMOID, f3 + p.db_bf);
      if (tpi == 1) {
        *reinterpret_cast<float2*>(top) = make_float2(s0, s1);
        *reinterpret_cast<float2*>(top + OW) = make_float2(s2, s3);
      } else if (tpi == 2) {
        *reinterpret_cast<float2*>(top + sub * OW) = sub ? make_float2(s2, s3) : make_float2(s0, s1);
      } else {
        top[(sub >> 1) * OW + (sub & 1)] = sub == 0 ? s0 : sub == 1 ? s1 : sub == 2 ? s2 : s3;
      }
    }
    return;
  }

  // Greedy-CTC classifier epilogue: each row's (max logit, sum of
  // exp(logit - max), last column holding the max) over this tile's columns.
  // TPR consecutive lanes share a row, each scanning CPT columns in order, so
  // ">=" keeps the last maximal column; lanes merge with xor shuffles.
  if (p.ctc_part) {
    constexpr int TPR = 256 / BM;
    constexpr int CPT = BN / TPR;
    const int row = tid / TPR, sub = tid % TPR;
    const int c0 = sub * CPT;
    const int nc = min(CPT, p.Co - (n0 + c0));  // valid columns of this lane
    const float* srow = row_ptr(row) + c0;
    const float* brow = p.bias + n0 + c0;
    float mx = -INFINITY, sum = 0.0f;
    int idx = -1;
    // Two passes over the staged row (LDS reads are cheap; holding the
    // logits in registers would cost the GEMM's occupancy).
#pragma unroll 4
    for (int c = 0; c < nc; ++c) {
      const float v = srow[c] + brow[c];
      if (v >= mx) {
        mx = v;
        idx = n0 + c0 + c;
      }
    }
#pragma unroll 4
    for (int c = 0; c < nc; ++c) sum += fast_exp(srow[c] + brow[c] - mx);
#pragma unroll
    for (int o = 1; o < TPR; o <<= 1) {
      const float om = __shfl_xor(mx, o), os = __shfl_xor(sum, o);
      const int oi = __shfl_xor(idx, o);
      lse_merge(mx, sum, idx, om, os, oi);
    }
    const int m = m0 + row;
    if (sub == 0 && m < M) {
      const size_t plane = (size_t)n_tiles * M;
      const size_t at = (size_t)(n0 / BN) * M + m;
      p.ctc_part[at] = mx;
      p.ctc_part[plane + at] = sum;
      p.ctc_part[2 * plane + at] = (float)idx;
    }
    return;
  }

  constexpr int NQ = BN / 4;
  const int col = staged_col<BN>(n0);
  const int row0 = tid / NQ;
  if ((p.out_ps & 3) == 0 && (p.Co & 3) == 0) {
    // Rows row0 + it * (256 / NQ) of column group col, two at a time: the
    // loads of both rows, then their stores (two rows bound the registers
    // held across the loads).
    constexpr int IT = BM * NQ / 256;
    constexpr int RSTEP = 256 / NQ;
    constexpr int CH = IT < 2 ? IT : 2;
    const bool need_coords = p.up != nullptr || p.rep != 1;
    const bool need_img = need_coords || p.res_gate != nullptr;
    const float4 b = bias_pre ? *bias_pre : bias4(p, col);
#pragma unroll
    for (int c0 = 0; c0 < IT; c0 += CH) {
      int img[CH], oy[CH], ox[CH];
      EpiTerms t[CH];
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int m = m0 + row0 + (c0 + c) * RSTEP;
        img[c] = oy[c] = ox[c] = 0;
        if (m >= M || col >= p.Co) continue;
        // Image and output coordinates only for the terms that use them
        // (the divisions would otherwise cost more than the rest of the
        // epilogue).
        if (need_img) {
          img[c] = m / HoWo;
          if (need_coords) {
            const int r = m - img[c] * HoWo;
            oy[c] = r / p.Wo;
            ox[c] = r - oy[c] * p.Wo;
          }
        }
        t[c] = epilogue_load<T>(p, m, col, img[c], oy[c], ox[c]);
      }
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int row = row0 + (c0 + c) * RSTEP;
        const int m = m0 + row;
        if (m >= M || col >= p.Co) continue;
        const float4 v = *reinterpret_cast<const float4*>(row_ptr(row) + (col - n0));
        epilogue_store<T>(p, v, b, t[c], m, col, img[c], oy[c], ox[c]);
      }
    }
    return;
  }
  // Channel counts that are not a multiple of 4 (the recognizer classifiers,
  // 6906 and 18710) carry no residual, gate or upsample terms.  An even Co
  // with fp32 output stores column pairs (8-byte aligned rows; half the
  // store instructions of element stores), anything else element by
  // element.
  if ((sizeof(T) == 4 || p.out_f32) && (p.out_ps & 1) == 0 && (p.Co & 1) == 0) {
    for (int row = row0; row < BM; row += 256 / NQ) {
      const int m = m0 + row;
      if (m >= M || col >= p.Co) continue;
      const float* v = row_ptr(row) + (col - n0);
      float* o = static_cast<float*>(p.out) + (size_t)m * p.out_ps + col;
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        if (col + e >= p.Co) break;
        float t0 = v[e], t1 = v[e + 1];
        if (p.bias) {
          t0 = t0 + p.bias[col + e];
          t1 = t1 + p.bias[col + e + 1];
        }
        *reinterpret_cast<float2*>(o + e) = make_float2(act_apply(p.act, t0), act_apply(p.act, t1));
      }
    }
    return;
  }
  for (int row = row0; row < BM; row += 256 / NQ) {
    const int m = m0 + row;
    if (m >= M || col >= p.Co) continue;
    const float* v = row_ptr(row) + (col - n0);
    for (int e = 0; e < 4 && col + e < p.Co; ++e) {
      float t = v[e];
      if (p.bias) t = t + p.bias[col + e];
      t = act_apply(p.act, t);
      size_t o = (size_t)m * p.out_ps + col + e;
      if (p.out_f32)
        static_cast<float*>(p.out)[o] = t;
      else
        st1<T>(static_cast<T*>(p.out) + o, t);
    }
  }
}

// Register epilogue (no LDS staging, no barrier).  An MFMA accumulator
// block holds, in lane l, column l % 16 of rows 4 (l / 16) .. +3; a 4x4
// transpose inside each quad of lanes (two DPP exchanges) turns that into
// row 4 (l / 16) + l % 4, columns 4 ((l % 16) / 4) .. +3, so each lane
// finishes whole float4 column groups and a quad stores 64 contiguous bytes
// of a row.  (Trading column blocks between lanes l and l ^ 32 so that one
// store writes whole 32-column rows measured slower.)

// quad_perm patterns of DPP: lane j reads lane j ^ 1, or lane j ^ 2.
constexpr int kDppXor1 = 0xB1;  // [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;  // [2, 3, 0, 1]

template <int CTRL>
__device__ __forceinline__ float dpp_swap(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Lane j of a quad holds a[e] = D[e][j] of a 4x4 block D; returns D[j][0..3].
// Every lane of the wave must be active.
__device__ __forceinline__ floatx4 quad_transpose(floatx4 a, int lane) {
  const bool odd = lane & 1;
  // Across lane bit 0: element e of lane j becomes D[e ^ 1][j ^ 1] where
  // e and j differ in bit 0.
  const float r0 = dpp_swap<kDppXor1>(odd ? a[0] : a[1]);
  const float r1 = dpp_swap<kDppXor1>(odd ? a[2] : a[3]);
  floatx4 b;
  b[0] = odd ? r0 : a[0];
  b[1] = odd ? a[1] : r0;
  b[2] = odd ? r1 : a[2];
  b[3] = odd ? a[3] : r1;
  // Across lane bit 1, element pairs (0, 2) and (1, 3).
  const bool hi = lane & 2;
  const float q0 = dpp_swap<kDppXor2>(hi ? b[0] : b[2]);
  const float q1 = dpp_swap<kDppXor2>(hi ? b[1] : b[3]);
  floatx4 c;
  c[0] = hi ? q0 : b[0];
  c[1] = hi ? q1 : b[1];
  c[2] = hi ? b[2] : q0;
  c[3] = hi ? b[3] : q1;
  return c;
}

// Column group of accumulator block column j of this lane after the quad
// transpose (finish_regs).
template <int BN, int WN>
__device__ __forceinline__ int regs_col(int n0, int j) {
  constexpr int TN = BN / (WN * 16);
  const int lane = threadIdx.x & 63;
  const int wn = (threadIdx.x >> 6) % WN;
  return n0 + wn * TN * 16 + j * 16 + 4 * ((lane & 15) >> 2);
}

// finish_tile without LDS: the split-K workspace store or the epilogue
// straight from the accumulators.  bias[j]: bias of column group
// regs_col(n0, j), loaded ahead.
// SE: also leave the SE channel sums of the stored output in p.se_part
// (single-image layers).
template <typename T, int BM, int BN, int WM, int WN, bool SE = false>
__device__ __forceinline__ void finish_regs(const ConvParams& p, floatx4 (&acc)[BM / (WM * 16)][BN / (WN * 16)],
                                            int m0, int n0, int M, const float4 (&bias)[BN / (WN * 16)]) {
  constexpr int TM = BM / (WM * 16);
  constexpr int TN = BN / (WN * 16);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WN;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = quad_transpose(acc[i][j], lane);
  const int rsub = 4 * (lane >> 4) + (lane & 3);
  if (p.splits > 1) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + wm * TM * 16 + i * 16 + rsub;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = regs_col<BN, WN>(n0, j);
        if (m < M && col < p.Co)
          *reinterpret_cast<float4*>(p.split_ws + ((size_t)blockIdx.y * M + m) * p.Co + col) =
              make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      }
    }
    return;
  }
  const int HoWo = p.Ho * p.Wo;
  const bool need_coords = p.up != nullptr || p.rep != 1;
  const bool need_img = need_coords || p.res_gate != nullptr;
  // SE channel sums (single image): this lane's rows of each column group,
  // then the wave's 16 row lanes of the group.
  float4 se_sum[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) se_sum[j] = float4{0.f, 0.f, 0.f, 0.f};
  // Row block by row block (the memory terms of a whole tile would cost the
  // main loop its occupancy): loads of the block's columns, then the stores.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * TM * 16 + i * 16 + rsub;
    if (m >= M) continue;
    int img = 0, oy = 0, ox = 0;
    if (need_img) {
      img = m / HoWo;
      if (need_coords) {
        const int r = m - img * HoWo;
        oy = r / p.Wo;
        ox = r - oy * p.Wo;
      }
    }
    EpiTerms t[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = regs_col<BN, WN>(n0, j);
      if (col < p.Co) t[j] = epilogue_load<T>(p, m, col, img, oy, ox);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = regs_col<BN, WN>(n0, j);
      if (col >= p.Co) continue;
      const float4 v = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      if ((p.Co & 3) != 0) {
        // Even Co, fp32 output, no epilogue terms (regs_epilogue): pairs.
        float4 x = p.bias ? f4_add(v, bias[j]) : v;
        x = make_float4(act_apply(p.act, x.x), act_apply(p.act, x.y), act_apply(p.act, x.z), act_apply(p.act, x.w));
        float* o = static_cast<float*>(p.out) + (size_t)m * p.out_ps + col;
        *reinterpret_cast<float2*>(o) = make_float2(x.x, x.y);
        if (col + 2 < p.Co) *reinterpret_cast<float2*>(o + 2) = make_float2(x.z, x.w);
        continue;
      }
      const float4 stored = epilogue_store<T>(p, v, bias[j], t[j], m, col, img, oy, ox);
      if constexpr (SE) se_sum[j] = f4_add(se_sum[j], stored);
    }
  }
  if constexpr (SE) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      float4 a = se_sum[j];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int o = k < 2 ? 1 << k : 1 << (k + 2);  // lane bits 0, 1, 4, 5: the rows of a column group
        a.x += __shfl_xor(a.x, o);
        a.y += __shfl_xor(a.y, o);
        a.z += __shfl_xor(a.z, o);
        a.w += __shfl_xor(a.w, o);
      }
      const int col = regs_col<BN, WN>(n0, j);
      if ((lane & 0x33) == 0 && col < p.Co)
        *reinterpret_cast<float4*>(p.se_part + ((size_t)(m0 / BM) * WM + wm) * p.Co + col) = a;
    }
  }
}

// DB head tail from registers (p.db_ch a multiple of 16, tiles whole taps
// wide).  After the quad transpose a lane holds row r and columns
// 4 g .. 4 g + 3 of a 16-column block, all in one tap (column tap * db_ch +
// o): it adds the bias, applies ReLU, multiplies by its four rows of
// conv_final's weights and adds the block's four column groups with xor
// shuffles.  The block partials go through LDS (`part`, BM x BN / 16
// float4, free once every wave has passed the barrier), and each (row, tap)
// item adds its db_ch / 16 blocks in order, applies the sigmoid and writes
// its 2x2 block of the map (src/cpu/model.rs:1516-1520).
template <typename T, int BM, int BN, int WM, int WN>
__device__ __forceinline__ void finish_db_regs(const ConvParams& p, floatx4 (&acc)[BM / (WM * 16)][BN / (WN * 16)],
                                               int m0, int n0, int M, const float4 (&bias)[BN / (WN * 16)],
                                               float4* part) {
  constexpr int TM = BM / (WM * 16);
  constexpr int TN = BN / (WN * 16);
  constexpr int NB = BN / 16;  // column blocks per tile
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int ch = p.db_ch;
  float4 wq[TN][4];  // conv_final weights of this lane's four hidden channels per block
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int o0 = regs_col<BN, WN>(n0, j) % ch;
#pragma unroll
    for (int e = 0; e < 4; ++e) wq[j][e] = *reinterpret_cast<const float4*>(p.db_wf + (size_t)(o0 + e) * 4);
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = quad_transpose(acc[i][j], lane);
  const int rsub = 4 * (lane >> 4) + (lane & 3);
  float4 f[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const float b[4] = {bias[j].x, bias[j].y, bias[j].z, bias[j].w};
      float4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float u = fmaxf(acc[i][j][e] + b[e], 0.0f);
        s.x = fmaf(u, wq[j][e].x, s.x);
        s.y = fmaf(u, wq[j][e].y, s.y);
        s.z = fmaf(u, wq[j][e].z, s.z);
        s.w = fmaf(u, wq[j][e].w, s.w);
      }
#pragma unroll
      for (int x = 4; x <= 8; x <<= 1) {
        s.x += __shfl_xor(s.x, x);
        s.y += __shfl_xor(s.y, x);
        s.z += __shfl_xor(s.z, x);
        s.w += __shfl_xor(s.w, x);
      }
      f[i][j] = s;
    }
  __syncthreads();  // every wave is done with the operand stages `part` overlays
  if (((lane >> 2) & 3) == 0) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) part[(wm * TM * 16 + i * 16 + rsub) * NB + wn * TN + j] = f[i][j];
  }
  __syncthreads();
  const int taps = BN / ch, per = ch / 16;
  const int HoWo = p.Ho * p.Wo;
  const int OW = 4 * p.Wo;
  float* map = static_cast<float*>(p.out);
  for (int it = tid; it < BM * taps; it += 256) {
    const int row = it / taps, tl = it - row * taps;
    const int m = m0 + row;
    if (m >= M) continue;
    float4 s = part[row * NB + tl * per];
    for (int b = 1; b < per; ++b) {
      const float4 t = part[row * NB + tl * per + b];
      s = make_float4(s.x + t.x, s.y + t.y, s.z + t.z, s.w + t.w);
    }
    const int img = m / HoWo, r = m - img * HoWo;
    const int y = r / p.Wo, x = r - y * p.Wo;
    const int tap = n0 / ch + tl;
    float* top = map + ((size_t)img * 4 * p.Ho + 4 * y + 2 * (tap >> 1)) * OW + 4 * x + 2 * (tap & 1);
    *reinterpret_cast<float2*>(top) =
        make_float2(act_apply(ACT_SIGMOID, s.x + p.db_bf), act_apply(ACT_SIGMOID, s.y + p.db_bf));
    *reinterpret_cast<float2*>(top + OW) =
        make_float2(act_apply(ACT_SIGMOID, s.z + p.db_bf), act_apply(ACT_SIGMOID, s.w + p.db_bf));
  }
}

// ---------------------------------------------------------------------------
// Direct-to-LDS variant (layers without an SE input gate, 16-byte k vectors).
// buffer_load_dwordx4 ... lds writes each lane's 16 bytes straight into LDS,
// so the operands never pass through registers and S K slices are in flight
// at once: slice s is multiplied while slices s+1 .. s+S-1 load.  The loads
// address the activation and weight tensors through buffer resources: lane
// offsets are 32-bit, and a masked lane (padding tap, row past M, k past K)
// gets an offset past the end of the buffer, which the hardware reads as
// zero.  For 1x1 layers a lane's offset is fixed for the whole K loop and
// the slice's k moves in the scalar offset, so the loop spends no vector
// instructions on addresses.  LDS rows are 64 bytes (one K slice of one
// tile row) with no padding; the four 16-byte vectors of row r are stored
// at positions v ^ swizzle_key(r), which makes the MFMA operand reads (lane
// l reads vector l / 16 of row l % 16) conflict-free.  A lane's LDS destination is fixed
// (base + 16 * lane), so the swizzle is applied by choosing which global
// vector each lane fetches.  The kernel orders its loads and LDS reads
// itself: explicit vmcnt waits before each barrier, and operand reads issued
// as inline assembly, which the compiler's wait insertion does not see (it
// would otherwise wait for every load in flight before each read).

// Offset past the end of every buffer the direct kernel reads (their sizes
// are checked below 2^31 bytes at launch): loads there return zero.
constexpr unsigned kOutOfRange = 0x80000000u;

__device__ void llvm_raw_buffer_load_lds(int32x4_t rsrc, __attribute__((address_space(3))) uint32_t* lds, int size,
                                         int voffset, int soffset, int offset,
                                         int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
__device__ u32x2 llvm_raw_buffer_load_v2i32(int32x4_t rsrc, int voffset, int soffset,
                                            int aux) __asm("llvm.amdgcn.raw.buffer.load.v2i32");
__device__ floatx4 llvm_raw_buffer_load_v4f32(int32x4_t rsrc, int voffset, int soffset,
                                              int aux) __asm("llvm.amdgcn.raw.buffer.load.v4f32");
__device__ void llvm_raw_buffer_store_v2i32(u32x2 v, int32x4_t rsrc, int voffset, int soffset,
                                            int aux) __asm("llvm.amdgcn.raw.buffer.store.v2i32");
typedef unsigned u32x4v __attribute__((ext_vector_type(4)));
__device__ u32x4v llvm_raw_buffer_load_v4i32(int32x4_t rsrc, int voffset, int soffset,
                                             int aux) __asm("llvm.amdgcn.raw.buffer.load.v4i32");
__device__ void llvm_raw_buffer_store_v4i32(u32x4v v, int32x4_t rsrc, int voffset, int soffset,
                                            int aux) __asm("llvm.amdgcn.raw.buffer.store.v4i32");
// ds_swizzle offset in its 32-lane bit-mask mode: lane l reads lane l ^ 4
// (and mask 0x1F, or mask 0, xor mask 4 in bits 10-14).
constexpr int kSwizzleXor4 = 0x1F | (4 << 10);

// One 16-byte buffer -> LDS load per lane from byte voffset + soffset of
// the resource (LDS destination base + 16 * lane, base wave-uniform).
__device__ __forceinline__ void lds_load16(int32x4_t rsrc, unsigned voffset, unsigned soffset, char* lds_base) {
  llvm_raw_buffer_load_lds(rsrc, (__attribute__((address_space(3))) uint32_t*)lds_base, 16, (int)voffset,
                           (int)soffset, 0, 0);
}

// Vector-position key of LDS row r (rows of 64 bytes, four 16-byte
// vectors): 2 * bit 2 of r.  Measured on this GPU with the LDS conflict
// counter (SQ_LDS_BANK_CONFLICT) for the operand read pattern: 4 cycles per
// ds_read_b128 with this key (a linear 16-byte-per-lane read also takes 4),
// against 8 for no swizzle and for the key (b2, b1 ^ b3) that is
// conflict-free when 8 or 16 consecutive lanes share a cycle.
__device__ __forceinline__ int swizzle_key(int r) { return ((r >> 2) & 1) << 1; }

typedef __attribute__((address_space(3))) void* lds_void_ptr;

// s_waitcnt with only the vector-memory count bounded (expcnt and lgkmcnt at
// their maxima): waits until at most N of this wave's loads are in flight.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Execution barrier without the memory fence of __syncthreads(), whose
// release would wait for every load in flight (vmcnt(0)) and so drain the
// pipeline.  The operand loads are ordered by the explicit vmcnt waits; the
// empty asm statements keep the compiler from moving LDS accesses across.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS offset of a __shared__ address.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// 16-byte LDS read issued as inline assembly; the value is usable only
// after lds_wait() on it.
__device__ __forceinline__ floatx4 lds_read16(unsigned addr) {
  floatx4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

// Waits for the LDS reads in flight; taking the value as an operand orders
// its uses after the wait.
__device__ __forceinline__ void lds_wait(floatx4& v) { asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v)); }

// GATE (fp32 1x1 layers whose tiles span at most two images): the SE gate
// rows of those images are staged in LDS once and each A operand fragment is
// multiplied by its gate values after it is read, x * g rounded to fp32 as
// when the gate is applied during the gather.
// Epilogue of the direct kernel, fixed per instantiation so each keeps only
// the registers its own epilogue needs.
enum DirectEpi : int {
  EPI_LDS = 0,      // finish_tile: staged through LDS (every epilogue)
  EPI_REGS = 1,     // finish_regs
  EPI_DB = 2,       // finish_db_regs (DB head tail)
  EPI_REGS_SE = 3,  // finish_regs leaving SE channel sums (fp32 1x1 layers with se_part)
};

// RB: bytes of one operand row per K slice, 64 (half a cache line, key
// swizzle_key) or 128 (a whole line, key direct_key<128>).
template <int RB>
__device__ __forceinline__ int direct_key(int r) {
  return RB == 64 ? swizzle_key(r) : (r >> 1) & 7;
}

// The direct kernel's work for output tile t of layer p (t in [0, M tiles x
// N tiles); other values return at once).
template <typename T, int BM, int BN, int WM, int WN, bool PW, int S, bool GATE, int EPI, int RB>
__device__ __forceinline__ void conv_gemm_direct_tile(const ConvParams& p, int t) {
  constexpr int BK = RB / sizeof(T);  // k values of one row per K slice
  constexpr int VE = 16 / sizeof(T);
  constexpr int TM = BM / (WM * 16);
  constexpr int TN = BN / (WN * 16);
  constexpr int LPR = RB / 16;     // load lanes per row
  constexpr int RPW = 64 / LPR;    // rows a wave fills per pass
  constexpr int RPP = 4 * RPW;     // rows a pass fills
  constexpr int H = RB / 64;       // 64-byte sub-slices (MFMA k steps of 16 fp32 / 32 bf16)
  static_assert(WM * WN == 4, "four waves per block");
  static_assert(BM % RPP == 0, "A rows load in whole passes");
  static_assert(S == 3 || S == 4, "three or four stages");
  static_assert(RB == 64 || RB == 128, "64- or 128-byte rows");
  constexpr int A_PASS = BM / RPP;
  constexpr int B_PASS = (BN + RPP - 1) / RPP;
  constexpr int STAGE_BYTES = (BM + BN) * RB;
  constexpr int LDE = BN + 4;
  constexpr int RPA = (BM + S - 1) / S;  // epilogue rows staged per stage array
  // The LDS epilogue stages the tile across the stage arrays; the others
  // need only the stages.
  constexpr int PART = EPI != EPI_LDS || STAGE_BYTES > RPA * LDE * 4 ? STAGE_BYTES : RPA * LDE * 4;
  __shared__ __attribute__((aligned(16))) char st0[PART];
  __shared__ __attribute__((aligned(16))) char st1[PART];
  __shared__ __attribute__((aligned(16))) char st2[PART];
  __shared__ __attribute__((aligned(16))) char st3[S == 4 ? PART : 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases and wait counts
  const int wm = wave / WN, wn = wave % WN;
  const int HoWo = p.Ho * p.Wo;
  // Stage j's LDS array (j is a constant at every call site once inlined).
  auto pick = [&](int j) -> char* { return j == 0 ? st0 : j == 1 ? st1 : j == 2 ? st2 : st3; };
  const int M = p.N * HoWo;
  const int K = p.kh * p.kw * p.C;
  constexpr int ES = sizeof(T);

  const int n_tiles = (p.Co + BN - 1) / BN;
  const int m_tiles = (M + BM - 1) / BM;
  if (t >= m_tiles * n_tiles) return;
  const int m0 = (t / n_tiles) * BM;
  const int n0 = (t % n_tiles) * BN;

  const int lrow = lane & 15;
  const int g = lane >> 4;

  // Gate rows of images img_lo and img_lo + 1: gate_lds[i] = gate of image
  // img_lo + i / C, channel i % C, zero past the gate array and in the BK
  // floats after both rows (read by the last slice's lanes past K).
  extern __shared__ __attribute__((aligned(16))) float gate_lds[];
  int g_sel[TM];  // first gate float of the image of A fragment i's row
  if constexpr (GATE) {
    const int img_lo = m0 / HoWo;
    const size_t g0 = (size_t)img_lo * p.C, gend = (size_t)p.N * p.C;
    for (int i = tid; i < 2 * p.C + BK; i += 256)
      gate_lds[i] = i < 2 * p.C && g0 + i < gend ? p.in_gate[g0 + i] : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = min(m0 + wm * TM * 16 + i * 16 + lrow, M - 1);
      g_sel[i] = (m / HoWo - img_lo) * p.C;
    }
    __syncthreads();
  }

  const int32x4_t a_rsrc = buffer_resource(p.in, (unsigned)((size_t)p.N * p.H * p.W * p.in_ps * ES));
  const int32x4_t b_rsrc = buffer_resource(p.wt, (unsigned)((size_t)p.Co * p.ldw * ES));

  // This lane fills LDS row pass * RPP + prow, position lane % LPR, with k
  // vector kvec of its source row: position ^ direct_key(row) (the key
  // depends on the row's low four bits only, and RPP is a multiple of 16).
  const int prow = wave * RPW + lane / LPR;
  const int kvec = (lane % LPR) ^ direct_key<RB>(prow);

  // Byte offsets of this lane's rows in the buffers (kOutOfRange for rows
  // past M or Co).  1x1: the row's k vector kvec, the slice's k0 goes in the
  // scalar offset.  Otherwise: the row's image; the tap is added per slice.
  unsigned a_off[A_PASS];
  int a_iy0[A_PASS], a_ix0[A_PASS];
#pragma unroll
  for (int i = 0; i < A_PASS; ++i) {
    const int m = m0 + i * RPP + prow;
    const bool ok = m < M;
    const int mm = ok ? m : 0;
    const int img = mm / HoWo;
    if constexpr (PW) {
      a_off[i] = ok ? (unsigned)(((size_t)mm * p.in_ps + kvec * VE) * ES) : kOutOfRange;
      a_iy0[i] = a_ix0[i] = 0;
    } else {
      const int r = mm - img * HoWo;
      const int oy = r / p.Wo;
      const int ox = r - oy * p.Wo;
      a_off[i] = ok ? (unsigned)((size_t)img * p.H * p.W * p.in_ps * ES) : kOutOfRange;
      a_iy0[i] = oy * p.sh - p.pt;
      a_ix0[i] = ox * p.sw - p.pl;
    }
  }
  unsigned b_off[B_PASS];
#pragma unroll
  for (int i = 0; i < B_PASS; ++i) {
    const int r = i * RPP + prow;
    const int n = n0 + r;
    b_off[i] = r < BN && n < p.Co ? (unsigned)(((size_t)n * p.ldw + kvec * VE) * ES) : kOutOfRange;
  }

  // K slices of this workgroup: all of them, or its split's share.
  const int nk_all = (K + BK - 1) / BK;
  const int s_begin = (int)((long)blockIdx.y * nk_all / gridDim.y);
  const int nk = (int)((long)(blockIdx.y + 1) * nk_all / gridDim.y) - s_begin;
  const int kbase = s_begin * BK;

  int kc = kbase + kvec * VE, kx = 0, ky = 0;
  if constexpr (!PW) {
    const int tap = kc / p.C;
    kc -= tap * p.C;
    ky = tap / p.kw;
    kx = tap - ky * p.kw;
  }

  // Issues the loads of the K slice at k0 (in order k0 = kbase,
  // kbase + BK, ...).  `tail`: the slice reaches past K, so lanes whose k
  // is past K are masked (only the last slice of a K that is not a multiple
  // of BK).
  auto issue_loads = [&](char* stage, int k0, auto tail) {
    constexpr bool TAIL = decltype(tail)::value;
    const unsigned ks = (unsigned)k0 * ES;
    const bool kin = !TAIL || k0 + kvec * VE < K;
#pragma unroll
    for (int i = 0; i < A_PASS; ++i) {
      char* dst = stage + (i * RPP + wave * RPW) * RB;
      if constexpr (PW) {
        lds_load16(a_rsrc, kin ? a_off[i] : kOutOfRange, ks, dst);
      } else {
        const int iy = a_iy0[i] + ky;
        const int ix = a_ix0[i] + kx;
        const bool ok = kin && a_off[i] != kOutOfRange && (unsigned)iy < (unsigned)p.H && (unsigned)ix < (unsigned)p.W;
        lds_load16(a_rsrc, ok ? a_off[i] + (unsigned)(((iy * p.W + ix) * p.in_ps + kc) * ES) : kOutOfRange, 0u,
                   dst);
      }
    }
#pragma unroll
    for (int i = 0; i < B_PASS; ++i)
      if (i * RPP + wave * RPW < BN)
        lds_load16(b_rsrc, kin ? b_off[i] : kOutOfRange, ks, stage + (BM + i * RPP + wave * RPW) * RB);
  };
  auto issue = [&](int j, int k0) {
    if (k0 + BK > K)
      issue_loads(pick(j), k0, std::true_type{});
    else
      issue_loads(pick(j), k0, std::false_type{});
    if constexpr (!PW) {
      kc += BK;
      while (kc >= p.C) {
        kc -= p.C;
        if (++kx == p.kw) {
          kx = 0;
          ++ky;
        }
      }
    }
  };

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Byte offset of this lane's vector in its row for sub-slice h: vector
  // g + 4 h (lane l reads vector l / 16 of row l % 16 in each 64-byte half).
  int swz[H];
#pragma unroll
  for (int h = 0; h < H; ++h) swz[h] = ((g + 4 * h) ^ direct_key<RB>(lrow)) << 4;

  // Operand reads go through lds_read16 (outside the compiler's view): the
  // compiler cannot tell the stage being read from the stages being filled
  // by the loads in flight and would otherwise wait for all of them before
  // every LDS read, draining the pipeline.  All sub-slices' reads are issued
  // before the first wait.
  auto compute = [&](int j, int k0) {
    const unsigned stage = lds_addr(pick(j));
    floatx4 ra[H][TM], rb[H][TN], gv[H][TM];
#pragma unroll
    for (int h = 0; h < H; ++h) {
#pragma unroll
      for (int i = 0; i < TM; ++i) ra[h][i] = lds_read16(stage + (wm * TM * 16 + i * 16 + lrow) * RB + swz[h]);
#pragma unroll
      for (int j = 0; j < TN; ++j) rb[h][j] = lds_read16(stage + (BM + wn * TN * 16 + j * 16 + lrow) * RB + swz[h]);
    }
    if constexpr (GATE) {
      // This lane's A values of sub-slice h are k0 + 16 h + 4g .. + 3 of its row.
#pragma unroll
      for (int h = 0; h < H; ++h)
#pragma unroll
        for (int i = 0; i < TM; ++i) gv[h][i] = lds_read16(lds_addr(gate_lds) + (g_sel[i] + k0 + 16 * h + 4 * g) * 4);
#pragma unroll
      for (int h = 0; h < H; ++h)
#pragma unroll
        for (int i = 0; i < TM; ++i) lds_wait(gv[h][i]);
    }
#pragma unroll
    for (int h = 0; h < H; ++h) {
#pragma unroll
      for (int i = 0; i < TM; ++i) lds_wait(ra[h][i]);
#pragma unroll
      for (int j = 0; j < TN; ++j) lds_wait(rb[h][j]);
    }
#pragma unroll
    for (int h = 0; h < H; ++h) {
      if constexpr (sizeof(T) == 4) {
        float4 a[TM], b[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = make_float4(ra[h][i][0], ra[h][i][1], ra[h][i][2], ra[h][i][3]);
        if constexpr (GATE) {
#pragma unroll
          for (int i = 0; i < TM; ++i)
            a[i] = make_float4(__fmul_rn(a[i].x, gv[h][i][0]), __fmul_rn(a[i].y, gv[h][i][1]),
                               __fmul_rn(a[i].z, gv[h][i][2]), __fmul_rn(a[i].w, gv[h][i][3]));
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) b[j] = make_float4(rb[h][j][0], rb[h][j][1], rb[h][j][2], rb[h][j][3]);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
      } else {
        bf16x8 a[TM], b[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = __builtin_bit_cast(bf16x8, ra[h][i]);
#pragma unroll
        for (int j = 0; j < TN; ++j) b[j] = __builtin_bit_cast(bf16x8, rb[h][j]);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
      }
    }
  };

  // One pipeline step: wait for slice s (slices s+1 .. s+S-2 may still be
  // loading), barrier (all waves' loads of slice s are in LDS and every wave
  // is done with slice s-1), refill the stage slice s-1 used with slice
  // s+S-1, multiply slice s.
  // Loads per wave per slice counted by the waits: the A passes, plus the B
  // passes when every wave takes part in them (BN >= RPP).  With BN < RPP
  // only some waves load B; counting A alone makes those waves wait a little
  // longer than needed, never less.
  constexpr int L = A_PASS + (BN >= RPP ? B_PASS : 0);
  auto step = [&](int cur, int refill, int s) {
    const int after = nk - 1 - s;  // slices issued after s (capped at S - 2)
    if (after >= S - 2)
      wait_vmcnt<(S - 2) * L>();
    else if (S == 4 && after == 1)
      wait_vmcnt<L>();
    else
      wait_vmcnt<0>();
    stage_barrier();
    if (s + S - 1 < nk) issue(refill, kbase + (s + S - 1) * BK);
    compute(cur, kbase + s * BK);
  };
  // Epilogue bias of this thread's column groups, loaded ahead so that its
  // latency hides behind the main loop.
  constexpr bool REGS = EPI != EPI_LDS;
  constexpr int NB = REGS ? TN : 1;
  float4 bias_pre[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int bcol = REGS ? regs_col<BN, WN>(n0, j) : staged_col<BN>(n0);
    bias_pre[j] = p.splits > 1 ? float4{0.f, 0.f, 0.f, 0.f} : bias4(p, bcol);
    // The last group of an even Co that is not a multiple of 4 has two columns.
    if (REGS && p.splits <= 1 && p.bias && bcol + 1 < p.Co && bcol + 3 >= p.Co)
      bias_pre[j] = make_float4(p.bias[bcol], p.bias[bcol + 1], 0.f, 0.f);
  }

  issue(0, kbase);
  if (nk > 1) issue(1, kbase + BK);
  if (S == 4 && nk > 2) issue(2, kbase + 2 * BK);
  for (int s = 0; s < nk; s += S) {
    if constexpr (S == 4) {
      step(0, 3, s);
      if (s + 1 < nk) step(1, 0, s + 1);
      if (s + 2 < nk) step(2, 1, s + 2);
      if (s + 3 < nk) step(3, 2, s + 3);
    } else {
      step(0, 2, s);
      if (s + 1 < nk) step(1, 0, s + 1);
      if (s + 2 < nk) step(2, 1, s + 2);
    }
  }
  wait_vmcnt<0>();  // every stage load has landed (the compiler does not count them all)
  if constexpr (EPI == EPI_DB) {
    static_assert(BM * (BN / 16) * 16 <= PART, "DB partials fit one stage");
    finish_db_regs<T, BM, BN, WM, WN>(p, acc, m0, n0, M, bias_pre, reinterpret_cast<float4*>(st0));
    return;
  }
  if constexpr (EPI == EPI_REGS || EPI == EPI_REGS_SE) {
    finish_regs<T, BM, BN, WM, WN, EPI == EPI_REGS_SE>(p, acc, m0, n0, M, bias_pre);
    return;
  }
  __syncthreads();

  finish_tile<T, BM, BN, WM, WN>(
      p, acc,
      [&](int row) {
        const int part = row / RPA;
        char* base = part == 0 ? st0 : part == 1 ? st1 : part == 2 ? st2 : st3;
        return reinterpret_cast<float*>(base) + (row - part * RPA) * LDE;
      },
      m0, n0, M, n_tiles, &bias_pre[0]);
}

// XCD-aware tile order (as conv_gemm_kernel): workgroup b takes tile
// (b % 8) * (grid / 8) + b / 8 (the grid is a multiple of 8).
__device__ __forceinline__ int xcd_tile() {
  const int per_xcd = gridDim.x / 8;
  return (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
}

template <typename T, int BM, int BN, int WM, int WN, bool PW, int S, bool GATE, int EPI, int RB = 64>
__global__ __launch_bounds__(256) void conv_gemm_direct_kernel(ConvParams p) {
  conv_gemm_direct_tile<T, BM, BN, WM, WN, PW, S, GATE, EPI, RB>(p, xcd_tile());
}

// Up to kConvMultiMax independent layers of one kernel instance in one
// launch (the FPN's per-level convs): the tiles of layer i follow those of
// layers 0 .. i - 1 in the XCD-aware order.
template <typename T, int BM, int BN, int WM, int WN, bool PW, int S, bool GATE, int EPI, int RB = 64>
__global__ __launch_bounds__(256) void conv_gemm_direct_multi_kernel(ConvMulti m) {
  int t = xcd_tile();
  int i = 0;
  while (i + 1 < m.count && t >= m.first[i + 1]) ++i;
  conv_gemm_direct_tile<T, BM, BN, WM, WN, PW, S, GATE, EPI, RB>(m.p[i], t - m.first[i]);
}

// ---------------------------------------------------------------------------
// Wide-tile bf16 1x1 layers (no SE input gate): 256x256 tiles, eight waves
// (2 x 4) of 128x64 each as 4 x 2 blocks of v_mfma_f32_32x32x16_bf16, so a
// tile multiplies 8.4 MFLOP per 64 KB K slice it stages: twice the operand
// reuse of the 128x64 tile, for the deep-K, wide-N layers whose MFMAs the
// smaller tiles' load latency starves.  One workgroup per CU: two LDS stages
// of 64-deep K slices, 128-byte rows (one cache line of each operand row per
// slice; 64-byte half-line rows measured 10-17 % slower: twice the L1
// requests per byte), filled by direct-to-LDS loads as in the kernel above
// while the other stage is multiplied; two waves per SIMD take turns on the
// matrix core.  The operand read of a 32x32x16 MFMA (lane l: 16 bytes of
// row l % 32, vector 2 kk + l / 32 of the row) is conflict-free with the
// row key (r / 2) % 8 (measured at the linear-read rate; without a key it
// runs at a sixth of it).  Epilogue from registers after the quad transpose.
//
// Persistent: the grid is one workgroup per CU, and each walks a run of
// tiles (those of its XCD's contiguous share, strided by the XCD's
// workgroup count, so the tiles in flight on one XCD share A row blocks in
// its L2).  The K-slice pipeline runs across tiles: the last slice of a tile
// issues the first slice of the next, and once every wave is done with the
// tile's last slice its stage takes the next tile's second slice; both load
// while the epilogue runs, and the epilogue's stores (every one issued, so
// counted) stay in flight across the next tile's first two waits.
// Cache policy (measured on the recognizer's layer shapes, isolated): the
// weights, re-read by every tile, should stay in L2 while the activations
// stream through it; layers without a residual store their outputs
// non-temporal and read A normally (1.15-1.19x against the non-persistent
// kernel), layers with a residual read A and the residual non-temporal and
// store normally (1.02-1.04x; the other way round they lose 3-9 %).  The
// epilogue overlap adds 1.08x on the GELU layers, 1.00-1.03x on the others.
constexpr int kWideBM = 256, kWideBN = 256;
constexpr int kAuxNontemporal = 2;  // cache-policy bit nt of the buffer load intrinsics

__device__ __forceinline__ int wide_key(int r) { return (r >> 1) & 7; }

typedef float floatx16 __attribute__((ext_vector_type(16)));

// Waits until at most N LDS reads of this wave are in flight; the six
// operands are the values whose reads must have completed (issued first).
template <int N>
__device__ __forceinline__ void lds_wait6(floatx4& a, floatx4& b, floatx4& c, floatx4& d, floatx4& e, floatx4& f) {
  asm volatile("s_waitcnt lgkmcnt(%6)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f) : "n"(N));
}

// RES: 0 no residual, 1 plain, 2 gated (res * res_gate of the row's image).
// F32OUT: fp32 output stored as float2 pairs (Co and out_ps even: the
// recognizer's classifier logits, 18710 columns, rows 8-byte aligned).
template <int RES, int ACT, bool F32OUT = false>
__global__ __launch_bounds__(512) void conv1x1_wide_kernel(ConvParams p) {
  constexpr int BM = kWideBM, BN = kWideBN, BK = 64;
  constexpr int WN = 4;          // 2 x 4 waves of 128x64
  constexpr int TM = 4, TN = 2;  // 32x32 blocks per wave
  constexpr int STAGE = (BM + BN) * 128;
  constexpr int ES = 2;
  constexpr int PASS = 64;  // rows one load pass of the 512 lanes fills (eight lanes per row)
  constexpr int AP = BM / PASS, BP = BN / PASS;
  __shared__ __attribute__((aligned(16))) char lds[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int M = p.N * p.Ho * p.Wo;
  const int K = p.C;

  const int n_tiles = (p.Co + BN - 1) / BN;
  const int m_tiles = (M + BM - 1) / BM;
  // Tiles of XCD x (workgroups b with b % 8 = x; the grid is a multiple of
  // 8): [x R, x R + R) with R = ceil(tiles / 8); its workgroup w = b / 8
  // takes tiles x R + w, x R + w + grid / 8, ...
  const int per_xcd = gridDim.x / 8;
  const int range = (m_tiles * n_tiles + 7) / 8;
  const int t_end = min(m_tiles * n_tiles, (int)(blockIdx.x % 8) * range + range);
  int t = (blockIdx.x % 8) * range + blockIdx.x / 8;
  if (t >= t_end) return;
  int m0 = (t / n_tiles) * BM;
  int n0 = (t % n_tiles) * BN;
  constexpr int AUX_A = RES != 0 ? kAuxNontemporal : 0;
  constexpr bool NT_STORE = RES == 0;

  const int32x4_t a_rsrc = buffer_resource(p.in, (unsigned)((size_t)p.N * p.H * p.W * p.in_ps * ES));
  const int32x4_t b_rsrc = buffer_resource(p.wt, (unsigned)((size_t)p.Co * p.ldw * ES));

  // Load lanes: lane fills row pass * PASS + prow, position lane % 8, with
  // k vector kvec of its source row.
  const int prow = wave * 8 + (lane >> 3);
  const int kvec = (lane & 7) ^ wide_key(prow);
  unsigned a_off[AP], b_off[BP];
  auto set_offsets = [&](int tm0, int tn0) {
#pragma unroll
    for (int i = 0; i < AP; ++i) {
      const int m = tm0 + i * PASS + prow;
      a_off[i] = m < M ? (unsigned)(((size_t)m * p.in_ps + kvec * 8) * ES) : kOutOfRange;
    }
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      const int n = tn0 + i * PASS + prow;
      b_off[i] = n < p.Co ? (unsigned)(((size_t)n * p.ldw + kvec * 8) * ES) : kOutOfRange;
    }
  };
  set_offsets(m0, n0);
  const int nk = (K + BK - 1) / BK;
  auto stage = [&](int j) { return lds + j * STAGE; };
  auto issue = [&](int j, int k0) {
    const unsigned ks = (unsigned)k0 * ES;
    const bool kin = k0 + kvec * 8 < K;
#pragma unroll
    for (int i = 0; i < AP; ++i)
      llvm_raw_buffer_load_lds(a_rsrc, (__attribute__((address_space(3))) uint32_t*)(stage(j) + (i * PASS + wave * 8) * 128),
                               16, (int)(kin ? a_off[i] : kOutOfRange), (int)ks, 0, AUX_A);
#pragma unroll
    for (int i = 0; i < BP; ++i)
      lds_load16(b_rsrc, kin ? b_off[i] : kOutOfRange, ks, stage(j) + (BM + i * PASS + wave * 8) * 128);
  };

  floatx16 acc[TM][TN];

  // Operand reads: row lane % 32 of each block, vector 2 kk + lane / 32 for
  // k step kk of the slice.  Two fragment sets alternate: the reads of k
  // step kk + 2 are issued once the MFMAs of step kk are, so they overlap
  // the MFMAs of step kk + 1 (the scheduling barriers keep each wait after
  // the MFMAs it follows).
  const int lr = lane & 31;
  const unsigned a_row = (unsigned)(wm * 128 + lr) * 128, b_row = (unsigned)(BM + wn * 64 + lr) * 128;
  unsigned swz[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) swz[kk] = (unsigned)((2 * kk + (lane >> 5)) ^ wide_key(lr)) << 4;
  auto compute = [&](int j) {
    const unsigned base = lds_addr(stage(j));
    floatx4 a0[TM], b0[TN], a1[TM], b1[TN];
    auto rd = [&](floatx4(&a)[TM], floatx4(&b)[TN], int kk) {
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = lds_read16(base + a_row + i * 32 * 128 + swz[kk]);
#pragma unroll
      for (int q = 0; q < TN; ++q) b[q] = lds_read16(base + b_row + q * 32 * 128 + swz[kk]);
    };
    auto mm = [&](floatx4(&a)[TM], floatx4(&b)[TN]) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int q = 0; q < TN; ++q)
          acc[i][q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[i]),
                                                               __builtin_bit_cast(bf16x8, b[q]), acc[i][q], 0, 0, 0);
    };
    rd(a0, b0, 0);
    rd(a1, b1, 1);
    lds_wait6<6>(a0[0], a0[1], a0[2], a0[3], b0[0], b0[1]);
    mm(a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    rd(a0, b0, 2);
    lds_wait6<6>(a1[0], a1[1], a1[2], a1[3], b1[0], b1[1]);
    mm(a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    rd(a1, b1, 3);
    lds_wait6<6>(a0[0], a0[1], a0[2], a0[3], b0[0], b0[1]);
    mm(a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    lds_wait6<0>(a1[0], a1[1], a1[2], a1[3], b1[0], b1[1]);
    mm(a1, b1);
  };
  // Vector memory operations of one lane's epilogue (residual loads, gate
  // loads, stores; all issued unconditionally, masked lanes by offset), and
  // of one slice's loads: the waits below count them.
  constexpr int E_OPS = (RES != 0 ? 16 : 0) + (RES == 2 ? 32 : 0) + (F32OUT ? 64 : 16);
  constexpr int LP = AP + BP;
  constexpr int W0 = LP + E_OPS < 63 ? LP + E_OPS : 63;
  constexpr int W1 = E_OPS < 63 ? E_OPS : 63;
  const int t_step = per_xcd;
  const bool has_bias = p.bias != nullptr;
  const int ccol = 4 * (lr >> 2);
  auto load_bias = [&](int tn0, float4 (&bias)[TN]) {
#pragma unroll
    for (int q = 0; q < TN; ++q) {
      const int col = tn0 + wn * 64 + q * 32 + ccol;
      bias[q] = bias4(p, col);
      if (F32OUT && p.bias && col + 1 < p.Co && col + 3 >= p.Co)
        bias[q] = make_float4(p.bias[col], p.bias[col + 1], 0.f, 0.f);
    }
  };
  float4 bias_cur[TN], bias_next[TN];
  load_bias(n0, bias_cur);
  wait_vmcnt<0>();  // the first tile's bias in registers before the pipeline starts
  bool first = true, pre1 = false;
  // Slice s of a tile: wait for its loads, barrier (every wave's loads of
  // slice s are in LDS and every wave is done reading slice s - 1), load
  // the next slice (s + 1, or the next tile's first) into the stage slice
  // s - 1 used, multiply.  The previous tile's epilogue operations are
  // younger than this tile's first two slices' loads, so those waits leave
  // them in flight.
  auto step = [&](int cur, int s, bool has_next) {
    if (s == 0 && !first)
      wait_vmcnt<W0>();
    else if (s == 1 && pre1)
      wait_vmcnt<W1>();
    else
      wait_vmcnt<0>();
    stage_barrier();
    if (s + 1 < nk) {
      if (!(s == 0 && pre1)) issue(cur ^ 1, (s + 1) * BK);
    } else if (has_next) {
      const int tn = t + t_step;
      set_offsets((tn / n_tiles) * BM, (tn % n_tiles) * BN);
      issue(cur ^ 1, 0);
    }
    // The next tile's bias loads here, long before the copy that waits for
    // them.
    if (s == 0 && has_next) load_bias(((t + t_step) % n_tiles) * BN, bias_next);
    compute(cur);
  };

  const int32x4_t out_rsrc = buffer_resource(p.out, (unsigned)((size_t)M * p.out_ps * (F32OUT ? 4 : 2)));
  const int32x4_t res_rsrc = buffer_resource(p.res, RES != 0 ? (unsigned)((size_t)M * p.res_ps * 2) : 0u);
  const int32x4_t gate_rsrc = buffer_resource(p.res_gate, RES == 2 ? (unsigned)((size_t)p.N * p.Co * 4) : 0u);
  issue(0, 0);
  int cur = 0;
  for (;;) {
    const bool has_next = t + t_step < t_end;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    for (int s = 0; s < nk; ++s) {
      step(cur, s, has_next);
      cur ^= 1;
    }
    // The next tile's second slice goes into the stage this tile's last
    // slice used, once every wave is done with it.
    pre1 = has_next && nk > 1;
    if (pre1) {
      stage_barrier();
      issue(cur ^ 1, BK);  // cur holds the next tile's first slice
    }
    first = false;

    // Epilogue: bias, activation, (gated) residual; the launcher sends the
    // other epilogue terms to the other kernels.  Block element e of lane l
    // is row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32; after the quad
    // transpose of elements 4 g .. 4 g + 3, lane l holds row 8 g + 4 (l / 32)
    // + l % 4, columns 4 ((l % 32) / 4) .. + 3 of each 32-column block.
    // Every residual, gate and store operation is issued (lanes past M or Co
    // masked by an out-of-range offset) so that the waits above can count
    // them; a row block's residual (and gate) loads are all issued before its
    // first store (a load cannot move above a store that may alias it).
    const int rsub = 4 * (lane >> 5) + (lane & 3);
    // Lanes l and l ^ 4 (column groups c and c ^ 1 of both blocks) move
    // whole 128-byte row lines between them: the even lane 8 columns of
    // block 0, the odd one 8 of block 1, starting at colw.
    const bool odd = (lane >> 2) & 1;
    const int colw = n0 + wn * 64 + (odd ? 32 : 0) + ((lr >> 2) & ~1) * 4;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      // Residual rows as whole lines: 16 bytes per lane at column colw, as
      // the stores below; lane l ^ 4 holds the other block's 4 columns.
      u32x4v rline[4];
      floatx4 rgate[4][TN];
      if constexpr (RES != 0) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int m = m0 + wm * 128 + i * 32 + 8 * g + rsub;
          const int img = RES == 2 ? min(m, M - 1) / (p.Ho * p.Wo) : 0;
          rline[g] = llvm_raw_buffer_load_v4i32(
              res_rsrc, m < M && colw < p.Co ? (int)(((size_t)m * p.res_ps + colw) * 2) : (int)kOutOfRange, 0,
              kAuxNontemporal);
          if constexpr (RES == 2) {
#pragma unroll
            for (int q = 0; q < TN; ++q) {
              const int col = n0 + wn * 64 + q * 32 + ccol;
              const bool ok = m < M && col < p.Co;
              rgate[g][q] = llvm_raw_buffer_load_v4f32(gate_rsrc, ok ? (int)(((size_t)img * p.Co + col) * 4) : (int)kOutOfRange,
                                                       0, 0);
            }
          }
        }
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 rq[TN];
        if constexpr (RES != 0) {
          const u32x2 keep = odd ? u32x2{rline[g][2], rline[g][3]} : u32x2{rline[g][0], rline[g][1]};
          const u32x2 give = odd ? u32x2{rline[g][0], rline[g][1]} : u32x2{rline[g][2], rline[g][3]};
          u32x2 got;
          got[0] = __builtin_amdgcn_ds_swizzle(give[0], kSwizzleXor4);
          got[1] = __builtin_amdgcn_ds_swizzle(give[1], kSwizzleXor4);
          rq[0] = odd ? got : keep;
          rq[1] = odd ? keep : got;
        }
        floatx4 v[TN];
#pragma unroll
        for (int q = 0; q < TN; ++q)
          v[q] = quad_transpose(floatx4{acc[i][q][4 * g], acc[i][q][4 * g + 1], acc[i][q][4 * g + 2], acc[i][q][4 * g + 3]},
                                lane);
        const int m = m0 + wm * 128 + i * 32 + 8 * g + rsub;
        u32x2 packed[TN];
#pragma unroll
        for (int q = 0; q < TN; ++q) {
          const int col = n0 + wn * 64 + q * 32 + ccol;
          float4 x = make_float4(v[q][0], v[q][1], v[q][2], v[q][3]);
          if (has_bias) x = f4_add(x, bias_cur[q]);
          x.x = act_apply(ACT, x.x);
          x.y = act_apply(ACT, x.y);
          x.z = act_apply(ACT, x.z);
          x.w = act_apply(ACT, x.w);
          if constexpr (RES != 0) {
            const u32x2 u = rq[q];
            float4 r = unpack_bf16x4(u[0], u[1]);
            if constexpr (RES == 2) {
              const floatx4 gt = rgate[g][q];
              r = make_float4(mul_rn(r.x, gt[0]), mul_rn(r.y, gt[1]), mul_rn(r.z, gt[2]), mul_rn(r.w, gt[3]));
            }
            x = f4_add(r, x);
          }
          if constexpr (F32OUT) {
            const bool mok = m < M;
            const size_t o = (size_t)m * p.out_ps + col;
            llvm_raw_buffer_store_v2f32(f32x2v{x.x, x.y}, out_rsrc, mok && col < p.Co ? (int)(o * 4) : (int)kOutOfRange, 0, 0);
            llvm_raw_buffer_store_v2f32(f32x2v{x.z, x.w}, out_rsrc, mok && col + 2 < p.Co ? (int)(o * 4 + 8) : (int)kOutOfRange,
                                        0, 0);
          } else {
            packed[q] = u32x2{pack_bf16x2(x.x, x.y), pack_bf16x2(x.z, x.w)};
          }
        }
        if constexpr (!F32OUT) {
          // Lanes l and l ^ 4 trade halves so that one 16-byte store per
          // lane writes each row's 64 columns (128 bytes, a whole line) at
          // once: 1.02-1.17x against 8-byte stores of half lines, which the
          // non-temporal stores also write to HBM as partial lines.  (Co and
          // out_ps are multiples of 8 here.)
          const u32x2 give = odd ? packed[0] : packed[1];
          u32x2 got;
          got[0] = __builtin_amdgcn_ds_swizzle(give[0], kSwizzleXor4);
          got[1] = __builtin_amdgcn_ds_swizzle(give[1], kSwizzleXor4);
          const u32x4v w4 = odd ? u32x4v{got[0], got[1], packed[1][0], packed[1][1]}
                                : u32x4v{packed[0][0], packed[0][1], got[0], got[1]};
          llvm_raw_buffer_store_v4i32(w4, out_rsrc,
                                      m < M && colw < p.Co ? (int)(((size_t)m * p.out_ps + colw) * 2) : (int)kOutOfRange,
                                      0, NT_STORE ? kAuxNontemporal : 0);
        }
      }
    }
    if (!has_next) break;
    t += t_step;
    m0 = (t / n_tiles) * BM;
    n0 = (t % n_tiles) * BN;
    for (int q = 0; q < TN; ++q) bias_cur[q] = bias_next[q];
  }
}

// Split-K finish: one workgroup per 16x64 output tile, one float4 of it per
// lane.  A lane issues the loads of all its split partials at once (the
// reduction is short and latency-bound), adds them in split order, stages
// the sum in LDS and the tile runs the epilogue.
constexpr int kMaxSplits = 16;
constexpr int kFinishBM = 16, kFinishBN = 64;

template <typename T>
__global__ __launch_bounds__(256) void conv_splitk_finish_kernel(ConvParams p) {
  constexpr int LDE = kFinishBN + 4;
  constexpr int NQ = kFinishBN / 4;
  static_assert(kFinishBM * NQ == 256, "one float4 per lane");
  __shared__ __attribute__((aligned(16))) float stage[kFinishBM * LDE];
  const int M = p.N * p.Ho * p.Wo;
  const int n_tiles = (p.Co + kFinishBN - 1) / kFinishBN;
  const int m0 = (int)(blockIdx.x / n_tiles) * kFinishBM;
  const int n0 = (int)(blockIdx.x % n_tiles) * kFinishBN;
  const size_t plane = (size_t)M * p.Co;
  const int row = threadIdx.x / NQ;
  const int c = (threadIdx.x % NQ) * 4;
  const int m = m0 + row;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (m < M && n0 + c < p.Co) {
    const float* src = p.split_ws + (size_t)m * p.Co + n0 + c;
    float4 part[kMaxSplits];
#pragma unroll
    for (int sp = 0; sp < kMaxSplits; ++sp)
      if (sp < p.splits) part[sp] = *reinterpret_cast<const float4*>(src + sp * plane);
#pragma unroll
    for (int sp = 0; sp < kMaxSplits; ++sp)
      if (sp < p.splits) v = f4_add(v, part[sp]);
  }
  *reinterpret_cast<float4*>(stage + row * LDE + c) = v;
  __syncthreads();
  finish_staged<T, kFinishBM, kFinishBN>(
      p, [&](int row) { return stage + row * LDE; }, m0, n0, M, n_tiles, nullptr);
}

// Kernel variant launch_conv runs for a layer (pointers are only tested for
// null and 16-byte alignment).
enum ConvVariant : int {
  CV_DIRECT_1X1 = 0,   // conv_gemm_direct_kernel, 1x1
  CV_DIRECT = 1,       // conv_gemm_direct_kernel, k x k / strided
  CV_DIRECT_GATE = 2,  // conv_gemm_direct_kernel, gated 1x1 (fp32)
  CV_REG_1X1 = 3,      // conv_gemm_kernel, 1x1, 16-byte loads
  CV_REG = 4,          // conv_gemm_kernel, 16-byte loads
  CV_REG_1X1_V4 = 5,   // conv_gemm_kernel, 1x1, 8-byte bf16 loads
  CV_REG_V4 = 6,       // conv_gemm_kernel, 8-byte bf16 loads
};

static int conv_variant(const ConvParams& p, int BM) {
  const int es = p.dt == DT_BF16 ? 2 : 4;
  const int ve16 = 16 / es;
  const bool pw = p.kh == 1 && p.kw == 1 && p.sh == 1 && p.sw == 1 && p.pt == 0 && p.pl == 0 && p.Ho == p.H &&
                  p.Wo == p.W;
  const bool aligned = reinterpret_cast<uintptr_t>(p.in) % 16 == 0 && reinterpret_cast<uintptr_t>(p.wt) % 16 == 0;
  const bool v16 = p.C % ve16 == 0 && p.in_ps % ve16 == 0 && p.ldw % ve16 == 0 && aligned;
  // The direct kernel's buffer offsets are 32-bit with kOutOfRange as the
  // masked offset: both buffers must stay below 2^31 bytes.
  const bool small = (size_t)p.N * p.H * p.W * p.in_ps * es < kOutOfRange && (size_t)p.Co * p.ldw * es < kOutOfRange;
  if (!p.in_gate && v16 && small) return pw ? CV_DIRECT_1X1 : CV_DIRECT;
  // Gated fp32 1x1 layers whose tiles span at most two images (an image has
  // at least BM pixels) and whose two gate rows fit in 32 KB of LDS.
  const size_t gate_bytes = (2 * (size_t)p.C + GemmTraits<float>::BK) * sizeof(float);
  if (es == 4 && p.in_gate && pw && v16 && small && p.Ho * p.Wo >= BM && gate_bytes <= 32768) return CV_DIRECT_GATE;
  // Register kernel: 16-byte loads need every vector of VE channels 16-byte
  // aligned (fp32 layers always have C % 4 == 0).
  const bool wide = es == 4 || (p.C % 8 == 0 && p.in_ps % 8 == 0 && p.ldw % 8 == 0 && aligned);
  if (pw) return wide ? CV_REG_1X1 : CV_REG_1X1_V4;
  return wide ? CV_REG : CV_REG_V4;
}

// Whether the direct kernel finishes its tiles from registers (finish_regs,
// or finish_db_regs for the DB head with 16-column taps) rather than through
// LDS (finish_tile): it can with whole float4 column groups (Co and out_ps
// multiples of 4) and without the greedy-CTC epilogue.  Measured on the
// detector and recognizer layers: the register epilogue is faster for fp32;
// for bf16 the LDS one, whose stores write whole 128-byte row segments
// where a register store writes 32 bytes of each of 16 rows (2-20 % per
// layer on the batch-8 detector, up to 2x for upsample-on-write at 8x8
// blocks).
static bool regs_epilogue(const ConvParams& p) {
  if (p.ctc_part) return false;
  if (p.db_ch) return p.db_ch % 16 == 0;
  if (p.dt != DT_F32) return false;
  // Even channel counts with an fp32 output and no epilogue terms (the
  // recognizer classifiers' logits, 6906 and 18710 columns) store column
  // pairs from registers.
  const bool pairs = p.Co % 2 == 0 && p.out_ps % 2 == 0 && !p.res && !p.up && p.rep == 1;
  return (p.Co % 4 == 0 && p.out_ps % 4 == 0 && p.rep == 1) || pairs;
}

// bf16 64x64 1x1 layers of deep K and at least 512 output channels (the
// detector's 13x23 and 26x46 levels) stage whole 128-byte rows (three
// stages): 1.06-1.1x per layer in the detector plan; shallower K, the
// other tiles and fp32 measured slower with the larger LDS footprint (fewer
// workgroups per CU), and so did the recognizer's 192-channel K = 768
// layers.
static bool rows128_layer(const ConvParams& p) {
  return p.dt == DT_BF16 && p.C >= 768 && p.Co >= 512 && p.splits <= 1 && !p.db_ch && !p.ctc_part;
}

// bf16 64x64 k x k layers of K >= 1024 whose channel count is a multiple
// of 64 (a 128-byte row then stays within one tap): 128-byte rows too (the
// detector head's 3x3 K = 2304 conv 1.18x, the stem's K = 1152 conv 1.04x
// at batch 8).
static bool rows128_kxk(const ConvParams& p) {
  return p.dt == DT_BF16 && p.kh * p.kw * p.C >= 1024 && p.C % 64 == 0 && p.splits <= 1 && !p.db_ch && !p.ctc_part;
}

template <typename T, int BM, int BN, int WM, int WN>
static void launch_tile_kernel(const ConvParams& p, dim3 grid, hipStream_t s) {
  // Stages: fp32 slices take long enough on the MFMAs that three cover the
  // load latency (and the smaller LDS footprint fits more workgroups per
  // CU); bf16 takes four where they fit in about 40 KB.
  constexpr int S = sizeof(T) == 2 && (BM + BN) * 64 <= 10240 ? 4 : 3;
  constexpr int VW = 16 / sizeof(T);  // k values per 16-byte load
  const bool regs = regs_epilogue(p);
  switch (conv_variant(p, BM)) {
    case CV_DIRECT_1X1:
      if constexpr (sizeof(T) == 2 && BM == 64 && BN == 64) {
        if (rows128_layer(p)) {  // K >= 768: the LDS epilogue (regs_epilogue)
          hipLaunchKernelGGL((conv_gemm_direct_kernel<T, BM, BN, WM, WN, true, 3, false, EPI_LDS, 128>), grid,
                             dim3(256), 0, s, p);
          break;
        }
      }
      if (regs && p.db_ch)
        hipLaunchKernelGGL((conv_gemm_direct_kernel<T, BM, BN, WM, WN, true, S, false, EPI_DB>), grid, dim3(256), 0,
                           s, p);
      else if (regs && p.se_part && sizeof(T) == 4)
        hipLaunchKernelGGL((conv_gemm_direct_kernel<T, BM, BN, WM, WN, true, S, false, EPI_REGS_SE>), grid, dim3(256),
                           0, s, p);
      else if (regs)
        hipLaunchKernelGGL((conv_gemm_direct_kernel<T, BM, BN, WM, WN, true, S, false, EPI_REGS>), grid, dim3(256), 0,
                           s, p);
      else
        hipLaunchKernelGGL((conv_gemm_direct_kernel<T, BM, BN, WM, WN, true, S, false, EPI_LDS>), grid, dim3(256), 0,
                           s, p);
      break;
    case CV_DIRECT:
      if constexpr (sizeof(T) == 2 && BM == 64 && BN == 64) {
        if (rows128_kxk(p)) {
          hipLaunchKernelGGL((conv_gemm_direct_kernel<T, BM, BN, WM, WN, false, 3, false, EPI_LDS, 128>), grid,
                             dim3(256), 0, s, p);
          break;
        }
      }
      if (regs && !p.db_ch)
        hipLaunchKernelGGL((conv_gemm_direct_kernel<T, BM, BN, WM, WN, false, S, false, EPI_REGS>), grid, dim3(256),
                           0, s, p);
      else
        hipLaunchKernelGGL((conv_gemm_direct_kernel<T, BM, BN, WM, WN, false, S, false, EPI_LDS>), grid, dim3(256), 0,
                           s, p);
      break;
    case CV_DIRECT_GATE:
      if constexpr (sizeof(T) == 4) {
        const unsigned lds = (unsigned)((2 * (size_t)p.C + GemmTraits<T>::BK) * sizeof(float));
        if (regs && !p.db_ch)
          hipLaunchKernelGGL((conv_gemm_direct_kernel<T, BM, BN, WM, WN, true, S, true, EPI_REGS>), grid, dim3(256),
                             lds, s, p);
        else
          hipLaunchKernelGGL((conv_gemm_direct_kernel<T, BM, BN, WM, WN, true, S, true, EPI_LDS>), grid, dim3(256),
                             lds, s, p);
      }
      break;
    case CV_REG_1X1:
      hipLaunchKernelGGL((conv_gemm_kernel<T, BM, BN, WM, WN, true, VW>), grid, dim3(256), 0, s, p);
      break;
    case CV_REG:
      hipLaunchKernelGGL((conv_gemm_kernel<T, BM, BN, WM, WN, false, VW>), grid, dim3(256), 0, s, p);
      break;
    case CV_REG_1X1_V4:
      hipLaunchKernelGGL((conv_gemm_kernel<T, BM, BN, WM, WN, true, 4>), grid, dim3(256), 0, s, p);
      break;
    default:
      hipLaunchKernelGGL((conv_gemm_kernel<T, BM, BN, WM, WN, false, 4>), grid, dim3(256), 0, s, p);
      break;
  }
}

template <typename T, int BM, int BN, int WM, int WN>
static void launch_tile(const ConvParams& p, int M, hipStream_t s) {
  // Grid rows of workgroups rounded up to a multiple of the 8 XCDs; surplus
  // workgroups exit before touching memory (see the tile order above).  With
  // split K, grid row y takes split y.  Upsample-on-write layers of short K
  // (the medium neck's intraclass conv_final, K = 32, writing each pixel as
  // a 2x2 to 8x8 block) recompute the tile once per replica row, grid layer
  // z writing output row z of every block: the few tiles of the deep levels
  // would otherwise store rep^2 copies each from a handful of CUs (the 8x8
  // level at batch 1: 5 workgroups storing 4.9 MB).
  const long tiles = (long)((M + BM - 1) / BM) * ((p.Co + BN - 1) / BN);
  const int splits = p.splits > 1 ? p.splits : 1;
  const int K = p.kh * p.kw * p.C;
  if (p.rep > 1 && splits == 1 && K <= 64 && !p.ctc_part && !p.db_ch) {
    ConvParams q = p;
    q.rep_split = 1;
    launch_tile_kernel<T, BM, BN, WM, WN>(q, dim3((unsigned)((tiles + 7) / 8 * 8), 1, (unsigned)p.rep), s);
    return;
  }
  launch_tile_kernel<T, BM, BN, WM, WN>(p, dim3((unsigned)((tiles + 7) / 8 * 8), (unsigned)splits), s);
  if (splits > 1) {
    const long fin = (long)((M + kFinishBM - 1) / kFinishBM) * ((p.Co + kFinishBN - 1) / kFinishBN);
    hipLaunchKernelGGL(conv_splitk_finish_kernel<T>, dim3((unsigned)fin), dim3(256), 0, s, p);
  }
}

// Layers conv1x1_wide_kernel runs: bf16 1x1 layers without an SE input
// gate, at least 256 output channels and K >= 512, whose 256x256 tiles
// number at least 128 (shape test, shared with the planner's split choice),
// with at most the bias, one of the activations the kernel is built for and
// a (gated) residual in the epilogue; K = 256 only with at least 480
// tiles.  Measured against the 128x64 / 64x64 kernel inside the recognizer
// and detector plans: 1.07-1.37x at K = 512 to 1536; at K = 256 1.1x on the
// recognizer's 960-tile layers but 0.92x on the detector's 300-tile ones, and
// 0.91-0.93x at K = 128 (a CU holds one wide tile, so nothing overlaps its
// short K loop's ramp and its epilogue); on isolated layers 0.57-0.85x on
// 70-76 tiles and 0.72-0.74x with 128 output channels, where half of each
// tile is empty.
constexpr int kWideMinTiles = 128, kWideMinK = 512, kWideMinCo = 256;
constexpr int kWideMinKShort = 256, kWideMinTilesShort = 480;

// Layers with an fp32 output (the recognizer's classifier logits: even Co,
// K >= 128, no residual) take the kernel from K = 128 on: their store
// stream bounds them, and the float2 register epilogue writes it 1.9x faster
// than the LDS epilogue the other kernels need for a Co that is not a
// multiple of 4 (18710 x 192 classifier: 486 -> 252 us in isolation).
constexpr int kWideMinKF32 = 128;

static bool wide_shape(int M, int Co, int K, int dt, bool f32out = false) {
  const long tiles = (long)((M + kWideBM - 1) / kWideBM) * ((Co + kWideBN - 1) / kWideBN);
  const bool deep = f32out ? K >= kWideMinKF32 : K >= kWideMinK || (K >= kWideMinKShort && tiles >= kWideMinTilesShort);
  return dt == DT_BF16 && Co % (f32out ? 2 : 4) == 0 && Co >= kWideMinCo && deep && tiles >= kWideMinTiles;
}

static bool wide_layer(const ConvParams& p) {
  const bool act = p.act == ACT_NONE || p.act == ACT_RELU || p.act == ACT_HSWISH || p.act == ACT_GELU;
  const bool f32 = p.out_f32 != 0;
  // Epilogue buffer offsets are 32-bit with kOutOfRange as the masked offset.
  const size_t M = (size_t)p.N * p.Ho * p.Wo;
  const bool small = M * p.out_ps * (f32 ? 4 : 2) < kOutOfRange && (!p.res || M * p.res_ps * 2 < kOutOfRange);
  // bf16 outputs are stored 16 bytes (8 columns) at a time.
  const bool whole8 = f32 || (p.Co % 8 == 0 && p.out_ps % 8 == 0);
  return act && small && whole8 && wide_shape(p.N * p.Ho * p.Wo, p.Co, p.C, p.dt, f32) &&
         conv_variant(p, 128) == CV_DIRECT_1X1 &&
         (!p.res_gate || p.res) && !p.up && p.rep == 1 && !(f32 && p.res) && !p.ctc_part && !p.db_ch &&
         p.splits <= 1 && p.out_ps % (f32 ? 2 : 4) == 0 && (!p.res || p.res_ps % 8 == 0);
}

// Tile shapes of the direct and register kernels, indexed by pick_tile
// (rows, columns, waves along the rows; four waves per workgroup).
constexpr int kTileBM[] = {256, 128, 128, 64, 64, 64};
constexpr int kTileBN[] = {16, 32, 64, 64, 16, 32};
constexpr int kTileWM[] = {4, 4, 2, 2, 4, 4};
constexpr const char* kTileName[] = {"256x16", "128x32", "128x64", "64x64", "64x16", "64x32"};

// Tile choice: narrow output channel counts get tall tiles so no MFMA
// column is wasted, except that layers of at most 16 (32) columns take
// 64-row tiles while 256-row (128-row) ones would not give every CU two
// (the tiny detector's 16-channel FPN convs at 19136 pixels: 75 workgroups
// of 256 rows, 299 of 64, 1.3-1.4x per layer and without the split of K the
// few big tiles needed; its stem and head convs at 832x1472 2.5 % of the
// pass; the 32-column tiles 0.6-2.2 % on every batch-1 plan and 0.2-0.6 %
// on the batch-8 detectors, where taller tiles stay faster from about two
// per CU).  Wide layers: fp32 takes 64x64 (its MFMA is slow enough that the
// smaller tile's occupancy wins); bf16 takes 128x64 when that still gives
// every CU several blocks (its faster MFMA needs the operand reuse of the
// taller tile).  Layers whose 64x64 tiles would number fewer than 1024
// (four per CU; the batch-1 plans' deeper stages, the batch-8 plans'
// deepest) take 64x32 tiles: twice the workgroups to overlap each other's
// load latency, for less operand reuse per tile (same-box A/B against
// 64x64 everywhere: recognizers at batch 1 1.09-1.15x, detectors at batch 1
// 1.03-1.08x, batch-8 detectors 1.00-1.03x, tiny recognizer R64 1.03x;
// thresholds of 256-768 tiles gave less, 1536 and 2048 lost 5-7 % on the
// medium detector at batch 1).
static int pick_tile(int M, int cols, int dt) {
  if (cols <= 16) return (M + 255) / 256 < 512 ? 4 : 0;
  if (cols <= 32) return (M + 127) / 128 < 512 ? 5 : 1;
  if (dt == DT_BF16 && (long)((M + 127) / 128) * ((cols + 63) / 64) >= 2048) return 2;
  if ((long)((M + 63) / 64) * ((cols + 63) / 64) < 1024) return 5;
  return 3;
}

std::string conv_kernel_name(const ConvParams& p) {
  if (wide_layer(p)) return "conv_gemm_bf16<256x256,1x1>";
  static const char* variants[] = {",1x1", "", ",1x1,gate", ",1x1,reg", ",reg", ",1x1,reg4", ",reg4"};
  const int t = pick_tile(p.N * p.Ho * p.Wo, p.Co, p.dt);
  const int v = conv_variant(p, kTileBM[t]);
  const bool r128 = t == 3 && ((v == CV_DIRECT_1X1 && rows128_layer(p)) || (v == CV_DIRECT && rows128_kxk(p)));
  return std::string(p.dt == DT_BF16 ? "conv_gemm_bf16<" : "conv_gemm<") + kTileName[t] + variants[v] +
         (r128 ? ",r128" : "") + ">";
}

int conv_se_blocks(const ConvParams& p) {
  if (p.N != 1 || p.splits > 1 || p.Co % 4 || p.out_ps % 4 || p.rep != 1 || p.db_ch || p.ctc_part || wide_layer(p) ||
      !regs_epilogue(p))
    return 0;
  const int M = p.Ho * p.Wo;
  const int t = pick_tile(M, p.Co, p.dt);
  if (conv_variant(p, kTileBM[t]) != CV_DIRECT_1X1) return 0;
  return (M + kTileBM[t] - 1) / kTileBM[t] * kTileWM[t];
}

int conv_tile_cols(int M, int cols, int dt) {
  return kTileBN[pick_tile(M, cols, dt)];
}

// Split K when the tiles fill fewer than 192 of the 256 CUs: enough splits
// for about two workgroups per CU.  Also when they give only one to two
// workgroups per CU (<= 560 tiles) and K is deep (>= 48 slices), where the
// CUs holding two tiles set the time: splits for about eight workgroups per
// CU (measured on the detector's 13x23 and 52x92 layers: 1.2-1.4x faster
// with the finish pass included; shallower K or more tiles measured
// slower).  fp32 layers keep that up to 640 tiles (the batch-1 medium
// detector's 104x184 3x3 layers with 64 output channels, 598 tiles: head
// conv_down 1.22x, stem3 1.11x; the same bf16 layers measured 0.7-0.8x
// split, their faster MFMAs leaving less to share), with splits for about
// four workgroups per CU (its 26x46 layers: 1024 -> 512 split 7 ways took
// 1.09x the unsplit time, 4 ways 1.01x; 13x23 896 -> 1792 4 ways 0.92x,
// 7 ways 0.96x).  Each split keeps at
// least 8 K slices (the load pipeline is 3-4 slices deep), at most 16
// splits.
int conv_split_k(int M, int Co, int K, int dt) {
  const int t = pick_tile(M, Co, dt);
  const long tiles = (long)((M + kTileBM[t] - 1) / kTileBM[t]) * ((Co + kTileBN[t] - 1) / kTileBN[t]);
  const int bk = dt == DT_BF16 ? GemmTraits<bf16>::BK : GemmTraits<float>::BK;
  const int nk = (K + bk - 1) / bk;
  if (Co % 4 != 0 || wide_shape(M, Co, K, dt)) return 1;
  long s;
  if (tiles < 192)
    s = (512 + tiles - 1) / tiles;
  else if (tiles <= (dt == DT_F32 ? 640 : 560) && nk >= 48)
    s = ((dt == DT_F32 ? 1024 : 2048) + tiles - 1) / tiles;
  else
    return 1;
  s = std::min<long>(s, nk / 8);
  s = std::min<long>(s, kMaxSplits);
  return s >= 2 ? (int)s : 1;
}

template <typename T, int I>
static void launch_tile_shape(const ConvParams& p, int M, hipStream_t s) {
  launch_tile<T, kTileBM[I], kTileBN[I], kTileWM[I], 4 / kTileWM[I]>(p, M, s);
}

int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

template <typename T>
static void launch_typed(const ConvParams& p, hipStream_t s) {
  int M = p.N * p.Ho * p.Wo;
  if constexpr (sizeof(T) == 2) {
    if (wide_layer(p)) {
      // One persistent workgroup per CU (a multiple of 8, one share per XCD).
      const long tiles = (long)((M + kWideBM - 1) / kWideBM) * ((p.Co + kWideBN - 1) / kWideBN);
      const dim3 grid((unsigned)std::min<long>((tiles + 7) / 8 * 8, std::max(8, device_cus() / 8 * 8)));
      auto go = [&](auto res, auto act) {
        if (p.out_f32) {
          if constexpr (decltype(res)::value == 0)
            hipLaunchKernelGGL((conv1x1_wide_kernel<0, decltype(act)::value, true>), grid, dim3(512), 0, s, p);
        } else {
          hipLaunchKernelGGL((conv1x1_wide_kernel<decltype(res)::value, decltype(act)::value>), grid, dim3(512), 0, s,
                             p);
        }
      };
      auto with_act = [&](auto res) {
        switch (p.act) {
          case ACT_RELU: go(res, std::integral_constant<int, ACT_RELU>{}); break;
          case ACT_HSWISH: go(res, std::integral_constant<int, ACT_HSWISH>{}); break;
          case ACT_GELU: go(res, std::integral_constant<int, ACT_GELU>{}); break;
          default: go(res, std::integral_constant<int, ACT_NONE>{}); break;
        }
      };
      if (p.res_gate)
        with_act(std::integral_constant<int, 2>{});
      else if (p.res)
        with_act(std::integral_constant<int, 1>{});
      else
        with_act(std::integral_constant<int, 0>{});
      return;
    }
  }
  switch (pick_tile(M, p.Co, p.dt)) {
    case 0: launch_tile_shape<T, 0>(p, M, s); break;
    case 1: launch_tile_shape<T, 1>(p, M, s); break;
    case 2: launch_tile_shape<T, 2>(p, M, s); break;
    case 3: launch_tile_shape<T, 3>(p, M, s); break;
    case 4: launch_tile_shape<T, 4>(p, M, s); break;
    default: launch_tile_shape<T, 5>(p, M, s); break;
  }
}

bool conv_multi_supported(const ConvParams* p, int count) {
  if (count < 1 || count > kConvMultiMax) return false;
  const std::string name = conv_kernel_name(p[0]);
  for (int i = 0; i < count; ++i) {
    const ConvParams& q = p[i];
    const int t = pick_tile(q.N * q.Ho * q.Wo, q.Co, q.dt);
    const int v = conv_variant(q, kTileBM[t]);
    if (q.dt != p[0].dt || q.splits > 1 || q.rep != 1 || q.db_ch || q.ctc_part || q.in_gate || wide_layer(q) ||
        (v != CV_DIRECT_1X1 && v != CV_DIRECT) || conv_kernel_name(q) != name ||
        regs_epilogue(q) != regs_epilogue(p[0]) || (q.se_part != nullptr) != (p[0].se_part != nullptr))
      return false;
  }
  return true;
}

// The instance launch_tile_kernel would pick for layer m.p[0] (which every
// layer shares), over all the layers' tiles.
template <typename T, int BM, int BN, int WM, int WN>
static void launch_multi_kernel(const ConvMulti& m, dim3 grid, hipStream_t s) {
  const ConvParams& p = m.p[0];
  constexpr int S = sizeof(T) == 2 && (BM + BN) * 64 <= 10240 ? 4 : 3;
  const bool regs = regs_epilogue(p);
  switch (conv_variant(p, BM)) {
    case CV_DIRECT_1X1:
      if constexpr (sizeof(T) == 2 && BM == 64 && BN == 64) {
        if (rows128_layer(p)) {
          hipLaunchKernelGGL((conv_gemm_direct_multi_kernel<T, BM, BN, WM, WN, true, 3, false, EPI_LDS, 128>), grid,
                             dim3(256), 0, s, m);
          return;
        }
      }
      if (regs && p.se_part && sizeof(T) == 4)
        hipLaunchKernelGGL((conv_gemm_direct_multi_kernel<T, BM, BN, WM, WN, true, S, false, EPI_REGS_SE>), grid,
                           dim3(256), 0, s, m);
      else if (regs)
        hipLaunchKernelGGL((conv_gemm_direct_multi_kernel<T, BM, BN, WM, WN, true, S, false, EPI_REGS>), grid,
                           dim3(256), 0, s, m);
      else
        hipLaunchKernelGGL((conv_gemm_direct_multi_kernel<T, BM, BN, WM, WN, true, S, false, EPI_LDS>), grid,
                           dim3(256), 0, s, m);
      return;
    case CV_DIRECT:
      if constexpr (sizeof(T) == 2 && BM == 64 && BN == 64) {
        if (rows128_kxk(p)) {
          hipLaunchKernelGGL((conv_gemm_direct_multi_kernel<T, BM, BN, WM, WN, false, 3, false, EPI_LDS, 128>),
                             grid, dim3(256), 0, s, m);
          return;
        }
      }
      if (regs)
        hipLaunchKernelGGL((conv_gemm_direct_multi_kernel<T, BM, BN, WM, WN, false, S, false, EPI_REGS>), grid,
                           dim3(256), 0, s, m);
      else
        hipLaunchKernelGGL((conv_gemm_direct_multi_kernel<T, BM, BN, WM, WN, false, S, false, EPI_LDS>), grid,
                           dim3(256), 0, s, m);
      return;
    default:
      throw std::runtime_error("launch_conv_multi: unsupported kernel variant");
  }
}

template <typename T>
static void launch_multi_typed(const ConvMulti& m, hipStream_t s) {
  const int t = pick_tile(m.p[0].N * m.p[0].Ho * m.p[0].Wo, m.p[0].Co, m.p[0].dt);
  long total = 0;
  for (int i = 0; i < m.count; ++i) {
    const ConvParams& q = m.p[i];
    total += (long)((q.N * q.Ho * q.Wo + kTileBM[t] - 1) / kTileBM[t]) * ((q.Co + kTileBN[t] - 1) / kTileBN[t]);
  }
  const dim3 grid((unsigned)((total + 7) / 8 * 8));
  switch (t) {
    case 0: launch_multi_kernel<T, kTileBM[0], kTileBN[0], kTileWM[0], 4 / kTileWM[0]>(m, grid, s); break;
    case 1: launch_multi_kernel<T, kTileBM[1], kTileBN[1], kTileWM[1], 4 / kTileWM[1]>(m, grid, s); break;
    case 2: launch_multi_kernel<T, kTileBM[2], kTileBN[2], kTileWM[2], 4 / kTileWM[2]>(m, grid, s); break;
    case 3: launch_multi_kernel<T, kTileBM[3], kTileBN[3], kTileWM[3], 4 / kTileWM[3]>(m, grid, s); break;
    case 4: launch_multi_kernel<T, kTileBM[4], kTileBN[4], kTileWM[4], 4 / kTileWM[4]>(m, grid, s); break;
    default: launch_multi_kernel<T, kTileBM[5], kTileBN[5], kTileWM[5], 4 / kTileWM[5]>(m, grid, s); break;
  }
}

void launch_conv_multi(const ConvMulti& mm, hipStream_t s) {
  if (!conv_multi_supported(mm.p, mm.count)) throw std::runtime_error("launch_conv_multi: layers cannot share a launch");
  ConvMulti m = mm;
  const int t = pick_tile(m.p[0].N * m.p[0].Ho * m.p[0].Wo, m.p[0].Co, m.p[0].dt);
  int first = 0;
  for (int i = 0; i < m.count; ++i) {
    const ConvParams& q = m.p[i];
    m.first[i] = first;
    first += ((q.N * q.Ho * q.Wo + kTileBM[t] - 1) / kTileBM[t]) * ((q.Co + kTileBN[t] - 1) / kTileBN[t]);
  }
  if (m.p[0].dt == DT_BF16)
    launch_multi_typed<bf16>(m, s);
  else
    launch_multi_typed<float>(m, s);
}

void launch_conv(const ConvParams& p, hipStream_t s) {
  if (p.dt == DT_BF16)
    launch_typed<bf16>(p, s);
  else
    launch_typed<float>(p, s);
}

}  // namespace ppocr
