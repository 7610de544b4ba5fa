// DB detector postprocess on the device: binarise, 8-connected components,
// per-component score and rotated-box fit, replacing the host loop of
// src/ocr.rs:723-790 (extract_detections) with collect_component
// (:1006-1054) and fit_rotated_box (:1056-1118).
//
// Components are labelled with a union-find over the pixels (each label
// points at a smaller pixel index; unions link roots with atomicMin, so
// every loop strictly decreases an index and ends).  Labels start at the
// first pixel of each horizontal run (a per-row max-scan), so only runs of
// neighbouring rows are united, one union per touching pair of runs; finds
// halve their path as they go.  The root of a component is its smallest
// raster index, which is the pixel the reference's raster scan starts its
// BFS from.  Component moments (count, sum of scores, sums of x, y, x^2, xy,
// y^2) are summed per thread over 8 consecutive pixels, then over the lanes
// of a wave that share a component, before one lane issues the atomics.
// Moments are accumulated in fp64, so the centre and covariance are at least
// as accurate as the reference's sequential fp32 sums.  Box extents use
// order-preserving integer atomics.
//
// Pixel p of image n is index n*H*W + y*W + x; only pixels inside the
// image's content rectangle take part.
#include <mutex>

#include "device_math.h"

namespace ppocr {

// Device scratch of ppocr_hip_db_postprocess_static, for callers that cannot
// allocate: the staged maps and the work arrays of one call live here.
// Every GPU holds its own copy at its own address; the name is only a host
// stand-in, so host code uses the address db_scratch returns.
constexpr size_t kDbScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kDbScratchBytes];

size_t db_scratch_bytes() { return kDbScratchBytes; }

std::mutex* db_scratch_mutex(int device) {
  static std::mutex mus[64];
  return device >= 0 && device < 64 ? &mus[device] : nullptr;
}

hipError_t db_scratch(int device, void** ptr) {
  static std::mutex mu;
  static void* cached[64] = {};
  if (device < 0 || device >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!cached[device]) {
    int current = 0;
    hipError_t e = hipGetDevice(&current);
    if (e != hipSuccess) return e;
    e = hipSetDevice(device);
    if (e != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t back = hipSetDevice(current);
    if (e != hipSuccess) return e;
    if (back != hipSuccess) return back;
    cached[device] = p;
  }
  *ptr = cached[device];
  return hipSuccess;
}

namespace {

constexpr int PPT = 8;  // pixels per thread in the moment and extent passes

__device__ __forceinline__ int load_label(const int* L, int i) {
  return __hip_atomic_load(L + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Root of x with path halving: each visited node is re-pointed at its
// grandparent (an ancestor, so the forest stays valid under concurrency).
__device__ __forceinline__ int find_root(int* L, int x) {
  int p = load_label(L, x);
  while (p != x) {
    const int gp = load_label(L, p);
    if (gp == p) return p;
    atomicMin(L + x, gp);
    x = gp;
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
// Slot of this lane among the lanes of its wave that ask for one (`want`):
// one atomic per wave on *counter instead of one per lane.
__device__ __forceinline__ int wave_claim(int* counter, bool want) {
  const uint64_t mask = __ballot(want);
  if (!want) return -1;
  const int leader = __ffsll((unsigned long long)mask) - 1;
  const int lane = threadIdx.x & 63;
  int base = 0;
  if (lane == leader) base = atomicAdd(counter, __popcll(mask));
  base = __shfl(base, leader);
  return base + __popcll(mask & ((1ull << lane) - 1));
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

// The next pixel's position (raster order over images).
__device__ __forceinline__ void advance(const DbParams& p, PixelPos& q) {
  if (++q.x == p.W) {
    q.x = 0;
    if (++q.y == p.H) {
      q.y = 0;
      ++q.n;
    }
  }
}

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
  if (threadIdx.x < 3) counters[threadIdx.x] = 0;
}

// One block per image row: label = index of the first pixel of the pixel's
// horizontal run of foreground (>= threshold, inside the content), else -1.
// The run start of a foreground pixel is the largest run start at or before
// it: a max-scan over the row (per-thread chunks, then across the block).
__global__ __launch_bounds__(256) void db_runs_kernel(DbParams p) {
  __shared__ int carry[256];
  const int row = blockIdx.x;
  const int n = row / p.H, y = row - n * p.H;
  const long base = (long)row * p.W;
  const int cw = y < p.content[2 * n + 1] ? p.content[2 * n] : 0;
  const int per = (p.W + 255) / 256;
  const int x0 = min(p.W, (int)threadIdx.x * per), x1 = min(p.W, x0 + per);
  auto fg = [&](int x) { return x < cw && p.prob[base + x] >= p.threshold; };
  int last = -1;
  bool finite = true;
  for (int x = x0; x < x1; ++x) {
    finite = finite && isfinite(p.prob[base + x]);
    if (fg(x) && (x == 0 || !fg(x - 1))) last = x;
  }
  // extract_detections rejects a map holding any non-finite value (also
  // outside the content area); counters[2] tells the host.
  if (!finite) atomicOr(&p.counters[2], 1);
  carry[threadIdx.x] = last;
  __syncthreads();
  for (int o = 1; o < 256; o <<= 1) {  // inclusive max-scan of the chunk maxima
    const int v = threadIdx.x >= (unsigned)o ? carry[threadIdx.x - o] : -1;
    __syncthreads();
    carry[threadIdx.x] = max(carry[threadIdx.x], v);
    __syncthreads();
  }
  int run = threadIdx.x > 0 ? carry[threadIdx.x - 1] : -1;
  for (int x = x0; x < x1; ++x) {
    const bool f = fg(x);
    if (f && (x == 0 || !fg(x - 1))) run = x;
    p.label[base + x] = f ? (int)(base + run) : -1;
  }
}

// Unites each run with the runs of the row above that touch it (8-connected:
// columns a-1 .. b+1 for a run [a, b]).  A foreground pixel at the start of
// its run unites with the upper run over column a (or a-1); every pixel x
// whose upper-right neighbour starts an upper run (up(x) background,
// up(x+1) foreground) unites with that run.  Together these reach every
// upper run overlapping a-1 .. b+1, once each.
__global__ __launch_bounds__(256) void db_union_kernel(DbParams p) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.total) return;
  // Foreground is label >= 0, which unions never change; the label values
  // themselves do change under concurrent unions, so run starts are found
  // from the mask, not from label == index.
  if (p.label[i] < 0) return;
  const PixelPos q = locate(p, i);
  if (q.y == 0) return;
  const int me = (int)i;
  const int cw = p.content[2 * q.n];
  const long up = i - p.W;
  const bool up_fg = p.label[up] >= 0;
  if (q.x == 0 || p.label[i - 1] < 0) {  // run start
    if (up_fg)
      unite(p.label, me, (int)up);
    else if (q.x > 0 && p.label[up - 1] >= 0)
      unite(p.label, me, (int)(up - 1));
  }
  if (!up_fg && q.x + 1 < cw && p.label[up + 1] >= 0) unite(p.label, me, (int)(up + 1));
}

// label = root; each root takes a component slot and clears its moments.
// No union runs any more, so the parent links are followed with plain loads
// (a link another thread has just shortened still points at an ancestor).
__global__ __launch_bounds__(256) void db_flatten_kernel(DbParams p) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  int parent = i < p.total ? p.label[i] : -1;
  int root = (int)i;
  if (parent >= 0)
    while (parent != root) {
      root = parent;
      parent = p.label[root];
    }
  // Every lane takes part in the wave's slot claim (ballot and shuffle).
  const int id = wave_claim(&p.counters[0], parent >= 0 && root == (int)i);
  if (parent < 0) return;
  if (root == (int)i) {
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
// Each thread sums PPT consecutive pixels; a change of component inside the
// chunk flushes the finished part with its own atomics (only at run ends),
// and the last part goes through the wave-level combine.
__device__ __forceinline__ void flush_moments(const DbParams& p, int id, int c, const double* v) {
  atomicAdd(&p.count[id], c);
#pragma unroll
  for (int k = 0; k < 6; ++k) atomicAdd(&p.moments[6 * (size_t)id + k], v[k]);
}

__global__ __launch_bounds__(256) void db_moments_kernel(DbParams p) {
  const long i0 = ((long)blockIdx.x * 256 + threadIdx.x) * PPT;
  const int lane = threadIdx.x & 63;
  int id = -1, c = 0;
  double v[6] = {0, 0, 0, 0, 0, 0};
  PixelPos q = locate(p, i0);
  for (long i = i0; i < i0 + PPT && i < p.total; ++i, advance(p, q)) {
    const int r = p.label[i];
    const int pid = r >= 0 ? p.slot[r] : -1;
    if (pid < 0 || pid >= p.max_comp) continue;
    if (pid != id) {
      if (id >= 0) flush_moments(p, id, c, v);
      id = pid;
      c = 0;
#pragma unroll
      for (int k = 0; k < 6; ++k) v[k] = 0.0;
    }
    const double x = q.x + 0.5, y = q.y + 0.5;
    c += 1;
    v[0] += (double)p.prob[i];
    v[1] += x;
    v[2] += y;
    v[3] += x * x;
    v[4] += x * y;
    v[5] += y * y;
  }
  // Up to two wave-level combines (a large component's pixels fill whole
  // waves); lanes still pending after them flush on their own.
  const bool active = id >= 0;
  uint64_t pending = __ballot(active);
  for (int round = 0; round < 2 && pending; ++round) {
    const int leader = __ffsll((unsigned long long)pending) - 1;
    const int lid = __shfl(id, leader);
    const bool mine = active && id == lid && ((pending >> lane) & 1);
    pending &= ~__ballot(mine);
    const int cs = wave_sum(mine ? c : 0);
    double s[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) s[k] = wave_sum(mine ? v[k] : 0.0);
    if (lane == leader) flush_moments(p, lid, cs, s);
  }
  if ((pending >> lane) & 1) flush_moments(p, id, c, v);
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

// Extents of each kept component along its axis and normal (PPT pixels per
// thread, then the wave-level combine, as the moments).
__device__ __forceinline__ void flush_extent(const DbParams& p, int id, const float* m) {
  int* e = p.extent + 4 * (size_t)id;
  atomicMin(&e[0], ordered(m[0]));
  atomicMax(&e[1], ordered(m[1]));
  atomicMin(&e[2], ordered(m[2]));
  atomicMax(&e[3], ordered(m[3]));
}

__global__ __launch_bounds__(256) void db_extent_kernel(DbParams p) {
  const long i0 = ((long)blockIdx.x * 256 + threadIdx.x) * PPT;
  const int lane = threadIdx.x & 63;
  int id = -1;
  float m[4] = {INFINITY, -INFINITY, INFINITY, -INFINITY};
  PixelPos q = locate(p, i0);
  for (long i = i0; i < i0 + PPT && i < p.total; ++i, advance(p, q)) {
    const int r = p.label[i];
    const int pid = r >= 0 ? p.slot[r] : -1;
    if (pid < 0 || pid >= p.max_comp || !p.keep[pid]) continue;
    if (pid != id) {
      if (id >= 0) flush_extent(p, id, m);
      id = pid;
      m[0] = m[2] = INFINITY;
      m[1] = m[3] = -INFINITY;
    }
    const float* g = p.geom + 8 * (size_t)id;
    const float dx = (float)q.x + 0.5f - g[0], dy = (float)q.y + 0.5f - g[1];
    const float a = dx * g[2] + dy * g[3];
    const float nrm = dx * (-g[3]) + dy * g[2];
    m[0] = fminf(m[0], a);
    m[1] = fmaxf(m[1], a);
    m[2] = fminf(m[2], nrm);
    m[3] = fmaxf(m[3], nrm);
  }
  const bool active = id >= 0;
  uint64_t pending = __ballot(active);
  for (int round = 0; round < 2 && pending; ++round) {
    const int leader = __ffsll((unsigned long long)pending) - 1;
    const int lid = __shfl(id, leader);
    const bool mine = active && id == lid && ((pending >> lane) & 1);
    pending &= ~__ballot(mine);
    float s[4];
    s[0] = wave_min(mine ? m[0] : INFINITY);
    s[1] = wave_max(mine ? m[1] : -INFINITY);
    s[2] = wave_min(mine ? m[2] : INFINITY);
    s[3] = wave_max(mine ? m[3] : -INFINITY);
    if (lane == leader) flush_extent(p, lid, s);
  }
  if ((pending >> lane) & 1) flush_extent(p, id, m);
}

// Unclipped box in content coordinates, mapped to the source image
// (DetectorTransform::map_*_to_source, src/ocr.rs:66-74), appended to the
// detection list as {x0, y0, .., x3, y3, score, image, root}.
__global__ __launch_bounds__(256) void db_emit_kernel(DbParams p) {
#pragma clang fp contract(off)
  const int id = blockIdx.x * 256 + threadIdx.x;
  const int n_comp = min(p.counters[0], p.max_comp);
  const bool emit = id < n_comp && p.keep[id];
  const int slot = wave_claim(&p.counters[1], emit);
  if (!emit) return;
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

const char* const kDbKernelNames[kDbKernels] = {"reset", "runs", "union", "flatten",
                                                 "moments", "axis", "extent", "emit"};

void launch_db_postprocess(const DbParams& p, hipStream_t s, hipEvent_t* marks) {
  const unsigned px_blocks = (unsigned)((p.total + 255) / 256);
  const unsigned chunk_blocks = (unsigned)((p.total + 256L * PPT - 1) / (256L * PPT));
  const unsigned comp_blocks = (unsigned)((p.max_comp + 255) / 256);
  int k = 0;
  auto mark = [&] {
    if (marks) (void)hipEventRecord(marks[k++], s);
  };
  mark();
  hipLaunchKernelGGL(db_reset_kernel, dim3(1), dim3(64), 0, s, p.counters);
  mark();
  hipLaunchKernelGGL(db_runs_kernel, dim3((unsigned)(p.N * p.H)), dim3(256), 0, s, p);
  mark();
  hipLaunchKernelGGL(db_union_kernel, dim3(px_blocks), dim3(256), 0, s, p);
  mark();
  hipLaunchKernelGGL(db_flatten_kernel, dim3(px_blocks), dim3(256), 0, s, p);
  mark();
  hipLaunchKernelGGL(db_moments_kernel, dim3(chunk_blocks), dim3(256), 0, s, p);
  mark();
  hipLaunchKernelGGL(db_axis_kernel, dim3(comp_blocks), dim3(256), 0, s, p);
  mark();
  hipLaunchKernelGGL(db_extent_kernel, dim3(chunk_blocks), dim3(256), 0, s, p);
  mark();
  hipLaunchKernelGGL(db_emit_kernel, dim3(comp_blocks), dim3(256), 0, s, p);
  mark();
}

}  // namespace ppocr
