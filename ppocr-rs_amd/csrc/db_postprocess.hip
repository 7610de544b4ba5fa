// DB detector postprocess on the device: binarise, 8-connected components,
// per-component score and rotated-box fit, replacing the host loop of
// src/ocr.rs:723-790 (extract_detections) with collect_component
// (:1006-1054) and fit_rotated_box (:1056-1118).
//
// Components are labelled with a union-find over the pixels (each label
// points at a smaller pixel index; unions link roots with atomicMin, so
// every loop strictly decreases an index and ends).  The root of a component
// is its smallest raster index, which is the pixel the reference's raster
// scan starts its BFS from.  Component moments (count, sum of scores, sums
// of x, y, x^2, xy, y^2) are reduced within each wave over lanes that share a
// component before one lane issues the atomics, so a large component costs
// one atomic per wave, not per pixel.  Moments are accumulated in fp64, so
// the centre and covariance are at least as accurate as the reference's
// sequential fp32 sums.  Box extents use order-preserving integer atomics.
//
// Pixel p of image n is index n*H*W + y*W + x; only pixels inside the
// image's content rectangle take part.
#include "device_math.h"

namespace ppocr {

namespace {

__device__ __forceinline__ int load_label(const int* L, int i) {
  return __hip_atomic_load(L + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int find_root(const int* L, int x) {
  int p = load_label(L, x);
  while (p != x) {
    x = p;
    p = load_label(L, x);
  }
  return x;
}

__device__ void unite(int* L, int a, int b) {
  while (true) {
    a = find_root(L, a);
    b = find_root(L, b);
    if (a == b) return;
    if (a > b) {
      int t = a;
      a = b;
      b = t;
    }
    const int old = atomicMin(L + b, a);
    if (old == b) return;
    b = old;
  }
}

// Float -> int mapping that preserves order (for atomicMin/atomicMax).
__device__ __forceinline__ int ordered(float f) {
  int i = __float_as_int(f);
  return i >= 0 ? i : i ^ 0x7fffffff;
}
__device__ __forceinline__ float unordered(int i) { return __int_as_float(i >= 0 ? i : i ^ 0x7fffffff); }

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = fminf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

struct PixelPos {
  int n, x, y;
  bool inside;
};

__device__ __forceinline__ PixelPos locate(const DbParams& p, long i) {
  PixelPos q;
  const long hw = (long)p.H * p.W;
  q.n = (int)(i / hw);
  const int r = (int)(i - (long)q.n * hw);
  q.y = r / p.W;
  q.x = r - q.y * p.W;
  q.inside = q.n < p.N && q.x < p.content[2 * q.n] && q.y < p.content[2 * q.n + 1];
  return q;
}

}  // namespace

__global__ void db_reset_kernel(int* counters) {
  if (threadIdx.x < 2) counters[threadIdx.x] = 0;
}

// label = own index for pixels >= threshold inside the content, else -1.
__global__ __launch_bounds__(256) void db_init_kernel(DbParams p) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.total) return;
  const PixelPos q = locate(p, i);
  p.label[i] = q.inside && p.prob[i] >= p.threshold ? (int)i : -1;
}

// Links each foreground pixel with its foreground neighbours to the left,
// upper-left, up and upper-right; with every pixel doing so, all eight
// neighbour pairs are covered.
__global__ __launch_bounds__(256) void db_union_kernel(DbParams p) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.total || p.label[i] < 0) return;
  const PixelPos q = locate(p, i);
  const int cw = p.content[2 * q.n];
  const int me = (int)i;
  if (q.x > 0 && p.label[i - 1] >= 0) unite(p.label, me, me - 1);
  if (q.y > 0) {
    const long up = i - p.W;
    if (q.x > 0 && p.label[up - 1] >= 0) unite(p.label, me, (int)(up - 1));
    if (p.label[up] >= 0) unite(p.label, me, (int)up);
    if (q.x + 1 < cw && p.label[up + 1] >= 0) unite(p.label, me, (int)(up + 1));
  }
}

// label = root; each root takes a component slot and clears its moments.
__global__ __launch_bounds__(256) void db_flatten_kernel(DbParams p) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.total || p.label[i] < 0) return;
  const int root = find_root(p.label, (int)i);
  if (root == (int)i) {
    const int id = atomicAdd(&p.counters[0], 1);
    p.slot[i] = id;
    if (id < p.max_comp) {
      p.count[id] = 0;
      for (int k = 0; k < 6; ++k) p.moments[6 * (size_t)id + k] = 0.0;
      p.root[id] = (int)i;
    }
  }
  // The root's own label is already final; writing it again is harmless.
  p.label[i] = root;
}

// Component moments: count, sum of scores, sums of x, y, x^2, xy, y^2 of the
// pixel centres (x + 0.5, y + 0.5).
__global__ __launch_bounds__(256) void db_moments_kernel(DbParams p) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const int lane = threadIdx.x & 63;
  int id = -1;
  if (i < p.total) {
    const int r = p.label[i];
    if (r >= 0) id = p.slot[r];
  }
  const bool active = id >= 0 && id < p.max_comp;
  double v[6] = {0, 0, 0, 0, 0, 0};
  if (active) {
    const PixelPos q = locate(p, i);
    const double x = q.x + 0.5, y = q.y + 0.5;
    v[0] = (double)p.prob[i];
    v[1] = x;
    v[2] = y;
    v[3] = x * x;
    v[4] = x * y;
    v[5] = y * y;
  }
  uint64_t pending = __ballot(active);
  while (pending) {
    const int leader = __ffsll((unsigned long long)pending) - 1;
    const int lid = __shfl(id, leader);
    const bool mine = active && id == lid && ((pending >> lane) & 1);
    pending &= ~__ballot(mine);
    const int c = wave_sum(mine ? 1 : 0);
    double s[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) s[k] = wave_sum(mine ? v[k] : 0.0);
    if (lane == leader) {
      atomicAdd(&p.count[lid], c);
#pragma unroll
      for (int k = 0; k < 6; ++k) atomicAdd(&p.moments[6 * (size_t)lid + k], s[k]);
    }
  }
}

// Per component: score and area filters, centre and principal axis
// (angle = atan2(2 cov_xy, cov_xx - cov_yy) / 2, axis turned to x >= 0 as
// src/ocr.rs:1070-1073), and cleared extents.
__global__ __launch_bounds__(256) void db_axis_kernel(DbParams p) {
  const int id = blockIdx.x * 256 + threadIdx.x;
  const int n_comp = min(p.counters[0], p.max_comp);
  if (id >= n_comp) return;
  const int cnt = p.count[id];
  const double* m = p.moments + 6 * (size_t)id;
  const float score = (float)(m[0] / (double)cnt);
  const bool keep = cnt >= p.min_area && score >= p.box_threshold;
  p.keep[id] = keep ? 1 : 0;
  if (!keep) return;
  const double cx = m[1] / cnt, cy = m[2] / cnt;
  const float cxx = (float)(m[3] - m[1] * cx), cxy = (float)(m[4] - m[1] * cy), cyy = (float)(m[5] - m[2] * cy);
  const float angle = 0.5f * atan2f(2.0f * cxy, cxx - cyy);
  float ax = cosf(angle), ay = sinf(angle);
  if (ax < 0.0f || (fabsf(ax) < 1.1920929e-7f && ay < 0.0f)) {
    ax = -ax;
    ay = -ay;
  }
  float* g = p.geom + 8 * (size_t)id;
  g[0] = (float)cx;
  g[1] = (float)cy;
  g[2] = ax;
  g[3] = ay;
  g[4] = score;
  int* e = p.extent + 4 * (size_t)id;
  e[0] = ordered(INFINITY);
  e[1] = ordered(-INFINITY);
  e[2] = ordered(INFINITY);
  e[3] = ordered(-INFINITY);
}

// Extents of each kept component along its axis and normal.
__global__ __launch_bounds__(256) void db_extent_kernel(DbParams p) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const int lane = threadIdx.x & 63;
  int id = -1;
  if (i < p.total) {
    const int r = p.label[i];
    if (r >= 0) id = p.slot[r];
  }
  bool active = id >= 0 && id < p.max_comp && p.keep[id];
  float a = 0.0f, nrm = 0.0f;
  if (active) {
    const PixelPos q = locate(p, i);
    const float* g = p.geom + 8 * (size_t)id;
    const float dx = (float)q.x + 0.5f - g[0], dy = (float)q.y + 0.5f - g[1];
    a = dx * g[2] + dy * g[3];
    nrm = dx * (-g[3]) + dy * g[2];
  }
  uint64_t pending = __ballot(active);
  while (pending) {
    const int leader = __ffsll((unsigned long long)pending) - 1;
    const int lid = __shfl(id, leader);
    const bool mine = active && id == lid && ((pending >> lane) & 1);
    pending &= ~__ballot(mine);
    const float amin = wave_min(mine ? a : INFINITY), amax = wave_max(mine ? a : -INFINITY);
    const float nmin = wave_min(mine ? nrm : INFINITY), nmax = wave_max(mine ? nrm : -INFINITY);
    if (lane == leader) {
      int* e = p.extent + 4 * (size_t)lid;
      atomicMin(&e[0], ordered(amin));
      atomicMax(&e[1], ordered(amax));
      atomicMin(&e[2], ordered(nmin));
      atomicMax(&e[3], ordered(nmax));
    }
  }
}

// Unclipped box in content coordinates, mapped to the source image
// (DetectorTransform::map_*_to_source, src/ocr.rs:66-74), appended to the
// detection list as {x0, y0, .., x3, y3, score, image, root}.
__global__ __launch_bounds__(256) void db_emit_kernel(DbParams p) {
#pragma clang fp contract(off)
  const int id = blockIdx.x * 256 + threadIdx.x;
  const int n_comp = min(p.counters[0], p.max_comp);
  if (id >= n_comp || !p.keep[id]) return;
  const float* g = p.geom + 8 * (size_t)id;
  const int* e = p.extent + 4 * (size_t)id;
  const float min_a = unordered(e[0]), max_a = unordered(e[1]);
  const float min_n = unordered(e[2]), max_n = unordered(e[3]);
  const float ax = g[2], ay = g[3], nx = -ay, ny = ax;
  const float axis_center = (min_a + max_a) * 0.5f;
  const float normal_center = (min_n + max_n) * 0.5f;
  const float half_axis = ((max_a - min_a + 1.0f) * p.unclip) * 0.5f;
  const float half_normal = ((max_n - min_n + 1.0f) * p.unclip) * 0.5f;
  const float cx = g[0] + (ax * axis_center + nx * normal_center);
  const float cy = g[1] + (ay * axis_center + ny * normal_center);
  const int root = p.root[id];
  const int n = root / (p.H * p.W);
  const float sw = (float)p.source[2 * n], sh = (float)p.source[2 * n + 1];
  const float cw = (float)p.content_scale[2 * n], ch = (float)p.content_scale[2 * n + 1];
  const int slot = atomicAdd(&p.counters[1], 1);
  float* o = p.out + 12 * (size_t)slot;
  const float sa[4] = {-1.0f, 1.0f, 1.0f, -1.0f}, sn[4] = {-1.0f, -1.0f, 1.0f, 1.0f};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float px = cx + (ax * (sa[k] * half_axis) + nx * (sn[k] * half_normal));
    const float py = cy + (ay * (sa[k] * half_axis) + ny * (sn[k] * half_normal));
    o[2 * k] = fminf(fmaxf(px * sw / cw, 0.0f), sw);
    o[2 * k + 1] = fminf(fmaxf(py * sh / ch, 0.0f), sh);
  }
  o[8] = g[4];
  o[9] = __int_as_float(n);
  o[10] = __int_as_float(root);
  o[11] = 0.0f;
}

void launch_db_postprocess(const DbParams& p, hipStream_t s) {
  const unsigned px_blocks = (unsigned)((p.total + 255) / 256);
  const unsigned comp_blocks = (unsigned)((p.max_comp + 255) / 256);
  hipLaunchKernelGGL(db_reset_kernel, dim3(1), dim3(64), 0, s, p.counters);
  hipLaunchKernelGGL(db_init_kernel, dim3(px_blocks), dim3(256), 0, s, p);
  hipLaunchKernelGGL(db_union_kernel, dim3(px_blocks), dim3(256), 0, s, p);
  hipLaunchKernelGGL(db_flatten_kernel, dim3(px_blocks), dim3(256), 0, s, p);
  hipLaunchKernelGGL(db_moments_kernel, dim3(px_blocks), dim3(256), 0, s, p);
  hipLaunchKernelGGL(db_axis_kernel, dim3(comp_blocks), dim3(256), 0, s, p);
  hipLaunchKernelGGL(db_extent_kernel, dim3(px_blocks), dim3(256), 0, s, p);
  hipLaunchKernelGGL(db_emit_kernel, dim3(comp_blocks), dim3(256), 0, s, p);
}

}  // namespace ppocr
