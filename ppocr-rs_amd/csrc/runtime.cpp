// Contexts, sessions and the C ABI (include/ppocr_hip.h).
//
// A context is one device, one stream and one activation arena shared by all
// of its models (the reference's shared workspace, src/gpu/runtime.rs:80-83,
// :1718-1730): the arena grows to the largest plan loaded on it.  A model's
// launch list is captured once into a hipGraph and replayed; the capture is
// redone whenever the arena had to move.
#include <chrono>
#include <cmath>
#include <cstring>
#include <thread>

#include "runtime.h"

namespace ppocr {

std::string& last_error() {
  static thread_local std::string message;
  return message;
}

namespace {

struct DeviceBuffer {
  void* ptr = nullptr;
  size_t bytes = 0;
  int device = 0;
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer() {
    if (ptr) {
      int cur = 0;
      (void)hipGetDevice(&cur);
      (void)hipSetDevice(device);
      (void)hipFree(ptr);
      (void)hipSetDevice(cur);
    }
  }
};

}  // namespace
}  // namespace ppocr

struct ppocr_hip_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;
  char* arena = nullptr;
  size_t arena_bytes = 0;
  uint64_t generation = 0;  // bumped whenever the arena moves
  ~ppocr_hip_ctx() {
    (void)hipSetDevice(device);
    if (stream) (void)hipStreamSynchronize(stream);
    if (arena) (void)hipFree(arena);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

struct ppocr_hip_model {
  ppocr_hip_ctx* ctx = nullptr;
  ppocr::Plan plan;
  size_t in_shape[4] = {0, 0, 0, 0};
  std::shared_ptr<ppocr::DeviceBuffer> weights;
  size_t weight_blob_bytes = 0;
  std::string weights_path;
  int size = 0;
  hipGraphExec_t graph = nullptr;
  uint64_t graph_generation = UINT64_MAX;
  ~ppocr_hip_model() {
    if (graph) (void)hipGraphExecDestroy(graph);
  }
};

struct ppocr_hip_image {
  ppocr_hip_ctx* ctx = nullptr;
  uint32_t width = 0, height = 0;
  std::shared_ptr<ppocr::DeviceBuffer> pixels;
};

namespace ppocr {
namespace {

std::shared_ptr<DeviceBuffer> device_alloc(int device, size_t bytes) {
  auto b = std::make_shared<DeviceBuffer>();
  b->device = device;
  b->bytes = bytes;
  if (bytes) HIP_OK(hipMalloc(&b->ptr, bytes));
  return b;
}

// Grows the shared arena to `bytes` (caller holds ctx->mu).
void ensure_arena(ppocr_hip_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->arena_bytes) return;
  HIP_OK(hipStreamSynchronize(ctx->stream));
  if (ctx->arena) HIP_OK(hipFree(ctx->arena));
  ctx->arena = nullptr;
  ctx->arena_bytes = 0;
  HIP_OK(hipMalloc(reinterpret_cast<void**>(&ctx->arena), bytes));
  ctx->arena_bytes = bytes;
  ++ctx->generation;
}

Exec exec_of(ppocr_hip_model* m) {
  Exec ex;
  ex.arena = m->ctx->arena;
  ex.weights = static_cast<const char*>(m->weights->ptr);
  ex.bufs = &m->plan.bufs;
  return ex;
}

void launch_all(ppocr_hip_model* m, hipStream_t s) {
  Exec ex = exec_of(m);
  for (const Op& op : m->plan.ops) op.launch(ex, s);
}

// Captures the launch list into a graph if the arena moved since the last
// capture (caller holds ctx->mu and has sized the arena).
void ensure_graph(ppocr_hip_model* m) {
  ppocr_hip_ctx* ctx = m->ctx;
  if (m->graph && m->graph_generation == ctx->generation) return;
  if (m->graph) {
    HIP_OK(hipGraphExecDestroy(m->graph));
    m->graph = nullptr;
  }
  hipGraph_t graph = nullptr;
  HIP_OK(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
  launch_all(m, ctx->stream);
  hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    raise(PPOCR_ERR_GPU, std::string("graph capture failed: ") + hipGetErrorString(e));
  }
  hipError_t ie = hipGraphInstantiate(&m->graph, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (ie != hipSuccess) raise(PPOCR_ERR_GPU, std::string("graph instantiate failed: ") + hipGetErrorString(ie));
  m->graph_generation = ctx->generation;
}

void check_input(ppocr_hip_model* m, const float* nchw, size_t len) {
  size_t expected = m->in_shape[0] * m->in_shape[1] * m->in_shape[2] * m->in_shape[3];
  if (!nchw) raise(PPOCR_ERR_INVALID_INPUT, "input pointer is null");
  if (len != expected)
    raise(PPOCR_ERR_INVALID_INPUT,
          "input has " + std::to_string(len) + " values; the planned shape needs " + std::to_string(expected));
  for (size_t i = 0; i < len; ++i)
    if (!std::isfinite(nchw[i])) raise(PPOCR_ERR_INVALID_INPUT, "input contains non-finite values");
}

// Device pointer of the plan's NCHW staging buffer / output buffer.
float* staging_ptr(ppocr_hip_model* m) {
  return reinterpret_cast<float*>(m->ctx->arena + m->plan.bufs[m->plan.staging].arena_off);
}
float* output_ptr(ppocr_hip_model* m) {
  return reinterpret_cast<float*>(m->ctx->arena + m->plan.bufs[m->plan.output].arena_off);
}

void upload_input(ppocr_hip_model* m, const float* nchw, size_t len) {
  HIP_OK(hipMemcpyAsync(staging_ptr(m), nchw, len * sizeof(float), hipMemcpyHostToDevice, m->ctx->stream));
}

void run_graph(ppocr_hip_model* m) { HIP_OK(hipGraphLaunch(m->graph, m->ctx->stream)); }

void read_output(ppocr_hip_model* m, float* out, size_t cap) {
  size_t n = m->plan.output_elems;
  if (!out || cap < n)
    raise(PPOCR_ERR_INVALID_INPUT, "output capacity " + std::to_string(cap) + " is below " + std::to_string(n));
  HIP_OK(hipMemcpyAsync(out, output_ptr(m), n * sizeof(float), hipMemcpyDeviceToHost, m->ctx->stream));
  HIP_OK(hipStreamSynchronize(m->ctx->stream));
  for (size_t i = 0; i < n; ++i)
    if (!std::isfinite(out[i])) raise(PPOCR_ERR_GPU, "model output contains non-finite values");
}

ppocr_hip_model* load_model(ppocr_hip_ctx* ctx, const char* path, ppocr_model_size size, const size_t nchw[4],
                            ppocr_precision precision, const ppocr_hip_model* share, bool detector,
                            bool greedy = false) {
  if (!ctx) raise(PPOCR_ERR_INVALID_INPUT, "context is null");
  if (!path) raise(PPOCR_ERR_INVALID_INPUT, "weights path is null");
  if (!nchw) raise(PPOCR_ERR_INVALID_INPUT, "input shape is null");
  if (size < PPOCR_SIZE_MEDIUM || size > PPOCR_SIZE_TINY) raise(PPOCR_ERR_INVALID_INPUT, "unknown model size");
  if (precision != PPOCR_F32 && precision != PPOCR_BF16) raise(PPOCR_ERR_INVALID_INPUT, "unknown precision");
  const int dt = precision == PPOCR_BF16 ? DT_BF16 : DT_F32;
  SafeTensors st = SafeTensors::load(path);
  auto m = std::make_unique<ppocr_hip_model>();
  m->ctx = ctx;
  m->size = size;
  m->weights_path = path;
  std::copy(nchw, nchw + 4, m->in_shape);
  m->plan = detector ? build_detector(st, size, nchw, dt) : build_recognizer(st, size, nchw, dt, greedy);
  m->weight_blob_bytes = m->plan.weights.size();
  std::lock_guard<std::mutex> lock(ctx->mu);
  HIP_OK(hipSetDevice(ctx->device));
  // The weight blob depends only on (file, tier, precision): the plan packs
  // the same tensors in the same order whatever the input shape.
  if (share && share->weights && share->size == size && share->weights_path == m->weights_path &&
      share->plan.dt == m->plan.dt && share->weight_blob_bytes == m->weight_blob_bytes) {
    m->weights = share->weights;
  } else {
    m->weights = device_alloc(ctx->device, m->weight_blob_bytes);
    HIP_OK(hipMemcpy(m->weights->ptr, m->plan.weights.data(), m->weight_blob_bytes, hipMemcpyHostToDevice));
  }
  std::vector<uint8_t>().swap(m->plan.weights);
  ensure_arena(ctx, m->plan.arena_bytes);
  return m.release();
}

}  // namespace
}  // namespace ppocr

using namespace ppocr;

extern "C" {

const char* ppocr_hip_last_error(void) { return last_error().c_str(); }

ppocr_status ppocr_hip_create(int device, ppocr_hip_ctx** out) {
  return guarded([&] {
    if (!out) raise(PPOCR_ERR_INVALID_INPUT, "output handle pointer is null");
    *out = nullptr;
    int count = 0;
    HIP_OK(hipGetDeviceCount(&count));
    if (device < 0 || device >= count)
      raise(PPOCR_ERR_GPU, "device " + std::to_string(device) + " not present (" + std::to_string(count) + " visible)");
    auto ctx = std::make_unique<ppocr_hip_ctx>();
    ctx->device = device;
    HIP_OK(hipSetDevice(device));
    HIP_OK(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
    *out = ctx.release();
  });
}

void ppocr_hip_destroy(ppocr_hip_ctx* ctx) { delete ctx; }

ppocr_status ppocr_hip_detector_load(ppocr_hip_ctx* ctx, const char* path, ppocr_model_size size, const size_t nchw[4],
                                     ppocr_precision precision, ppocr_hip_model** out) {
  return guarded([&] {
    if (!out) raise(PPOCR_ERR_INVALID_INPUT, "output handle pointer is null");
    *out = nullptr;
    *out = load_model(ctx, path, size, nchw, precision, nullptr, true);
  });
}

ppocr_status ppocr_hip_recognizer_load(ppocr_hip_ctx* ctx, const char* path, ppocr_model_size size,
                                       const size_t nchw[4], ppocr_precision precision,
                                       const ppocr_hip_model* share_weights, ppocr_hip_model** out) {
  return guarded([&] {
    if (!out) raise(PPOCR_ERR_INVALID_INPUT, "output handle pointer is null");
    *out = nullptr;
    if (share_weights && share_weights->plan.detector)
      raise(PPOCR_ERR_INVALID_INPUT, "shared weights must come from a recognizer");
    *out = load_model(ctx, path, size, nchw, precision, share_weights, false);
  });
}

ppocr_status ppocr_hip_recognizer_load_greedy(ppocr_hip_ctx* ctx, const char* path, ppocr_model_size size,
                                              const size_t nchw[4], ppocr_precision precision,
                                              const ppocr_hip_model* share_weights, ppocr_hip_model** out) {
  return guarded([&] {
    if (!out) raise(PPOCR_ERR_INVALID_INPUT, "output handle pointer is null");
    *out = nullptr;
    if (share_weights && share_weights->plan.detector)
      raise(PPOCR_ERR_INVALID_INPUT, "shared weights must come from a recognizer");
    *out = load_model(ctx, path, size, nchw, precision, share_weights, false, true);
  });
}

void ppocr_hip_model_free(ppocr_hip_model* model) {
  if (!model) return;
  std::lock_guard<std::mutex> lock(model->ctx->mu);
  (void)hipStreamSynchronize(model->ctx->stream);
  delete model;
}

ppocr_status ppocr_hip_output_shape(const ppocr_hip_model* model, size_t shape[4], size_t* rank) {
  return guarded([&] {
    if (!model || !shape || !rank) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    *rank = model->plan.output_shape.size();
    for (size_t i = 0; i < 4; ++i) shape[i] = i < *rank ? model->plan.output_shape[i] : 0;
  });
}

ppocr_status ppocr_hip_forward(ppocr_hip_model* model, const float* nchw, size_t len, float* out, size_t out_cap) {
  return guarded([&] {
    if (!model) raise(PPOCR_ERR_INVALID_INPUT, "model is null");
    check_input(model, nchw, len);
    std::lock_guard<std::mutex> lock(model->ctx->mu);
    HIP_OK(hipSetDevice(model->ctx->device));
    ensure_arena(model->ctx, model->plan.arena_bytes);
    ensure_graph(model);
    upload_input(model, nchw, len);
    run_graph(model);
    read_output(model, out, out_cap);
  });
}

ppocr_status ppocr_hip_upload_rgb(ppocr_hip_ctx* ctx, uint32_t width, uint32_t height, const uint8_t* rgb, size_t len,
                                  ppocr_hip_image** out) {
  return guarded([&] {
    if (!ctx || !out) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    *out = nullptr;
    if (width == 0 || height == 0) raise(PPOCR_ERR_INVALID_INPUT, "image dimensions must be positive");
    size_t bytes = (size_t)width * height * 3;
    if (!rgb || len != bytes)
      raise(PPOCR_ERR_INVALID_INPUT, "RGB image needs " + std::to_string(bytes) + " bytes, got " + std::to_string(len));
    std::lock_guard<std::mutex> lock(ctx->mu);
    HIP_OK(hipSetDevice(ctx->device));
    auto img = std::make_unique<ppocr_hip_image>();
    img->ctx = ctx;
    img->width = width;
    img->height = height;
    img->pixels = device_alloc(ctx->device, (bytes + 3) / 4 * 4);
    HIP_OK(hipMemcpy(img->pixels->ptr, rgb, bytes, hipMemcpyHostToDevice));
    *out = img.release();
  });
}

void ppocr_hip_image_free(ppocr_hip_image* image) { delete image; }

}  // extern "C"

namespace ppocr {
namespace {

// Runs the device preprocessing of `n` geometries into `dst` (fp32 NCHW
// planes).  Caller holds ctx->mu.
void run_preprocess(ppocr_hip_ctx* ctx, const ppocr_hip_image* image, const float* corners, const int* content_w,
                    int n, int cw, int ch, bool detector, float* dst) {
  static const float det_mean[3] = {0.485f, 0.456f, 0.406f}, det_std[3] = {0.229f, 0.224f, 0.225f};
  static const float rec_mean[3] = {0.5f, 0.5f, 0.5f}, rec_std[3] = {0.5f, 0.5f, 0.5f};
  const float* mean = detector ? det_mean : rec_mean;
  const float* stdv = detector ? det_std : rec_std;
  // Geometry table: corners [n][8] then content widths [n].
  size_t geo_bytes = (size_t)n * 8 * sizeof(float) + (size_t)n * sizeof(int);
  auto geo = device_alloc(ctx->device, geo_bytes);
  std::vector<char> host(geo_bytes);
  memcpy(host.data(), corners, (size_t)n * 8 * sizeof(float));
  memcpy(host.data() + (size_t)n * 8 * sizeof(float), content_w, (size_t)n * sizeof(int));
  HIP_OK(hipMemcpyAsync(geo->ptr, host.data(), geo_bytes, hipMemcpyHostToDevice, ctx->stream));
  PreParams p{};
  p.rgb = static_cast<const uint32_t*>(image->pixels->ptr);
  p.sw = (int)image->width;
  p.sh = (int)image->height;
  p.corners = static_cast<const float*>(geo->ptr);
  p.content_w = reinterpret_cast<const int*>(static_cast<const char*>(geo->ptr) + (size_t)n * 8 * sizeof(float));
  p.N = n;
  p.cw = cw;
  p.ch = ch;
  for (int c = 0; c < 3; ++c) {
    p.scale[c] = 1.0f / (255.0f * stdv[c]);
    p.bias[c] = -mean[c] / stdv[c];
  }
  p.out = dst;
  launch_preprocess(p, ctx->stream);
  HIP_OK(hipGetLastError());
  HIP_OK(hipStreamSynchronize(ctx->stream));
}

std::vector<int> content_widths(const size_t* widths, size_t n, size_t canvas) {
  std::vector<int> cw(n);
  for (size_t i = 0; i < n; ++i) {
    size_t w = widths ? widths[i] : canvas;
    if (w == 0 || w > canvas) raise(PPOCR_ERR_INVALID_INPUT, "content width outside 1..=canvas width");
    cw[i] = (int)w;
  }
  return cw;
}

void check_corners(const float* corners, size_t n) {
  if (!corners) raise(PPOCR_ERR_INVALID_INPUT, "corners pointer is null");
  for (size_t i = 0; i < n * 8; ++i)
    if (!std::isfinite(corners[i])) raise(PPOCR_ERR_INVALID_INPUT, "corners contain non-finite values");
}

}  // namespace
}  // namespace ppocr

extern "C" {

ppocr_status ppocr_hip_forward_image(ppocr_hip_model* model, const ppocr_hip_image* image, const float* corners,
                                     const size_t* content_w, size_t n, float* out, size_t out_cap) {
  return guarded([&] {
    if (!model || !image) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    if (image->ctx != model->ctx) raise(PPOCR_ERR_INVALID_INPUT, "image and model belong to different contexts");
    if (n != model->in_shape[0])
      raise(PPOCR_ERR_INVALID_INPUT, "geometry count " + std::to_string(n) + " differs from the planned batch");
    check_corners(corners, n);
    std::vector<int> cw = content_widths(content_w, n, model->in_shape[3]);
    std::lock_guard<std::mutex> lock(model->ctx->mu);
    HIP_OK(hipSetDevice(model->ctx->device));
    ensure_arena(model->ctx, model->plan.arena_bytes);
    ensure_graph(model);
    // Preprocess straight into the NCHW staging buffer the graph starts from.
    run_preprocess(model->ctx, image, corners, cw.data(), (int)n, (int)model->in_shape[3], (int)model->in_shape[2],
                   model->plan.detector, staging_ptr(model));
    run_graph(model);
    read_output(model, out, out_cap);
  });
}

ppocr_status ppocr_hip_preprocess(ppocr_hip_ctx* ctx, const ppocr_hip_image* image, const float corners[8],
                                  size_t canvas_w, size_t canvas_h, size_t content_width, int detector,
                                  float* out_nchw) {
  return guarded([&] {
    if (!ctx || !image || !out_nchw) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    if (canvas_w == 0 || canvas_h == 0 || canvas_w > (1u << 15) || canvas_h > (1u << 15))
      raise(PPOCR_ERR_INVALID_INPUT, "canvas dimensions out of range");
    check_corners(corners, 1);
    std::vector<int> cw = content_widths(&content_width, 1, canvas_w);
    std::lock_guard<std::mutex> lock(ctx->mu);
    HIP_OK(hipSetDevice(ctx->device));
    size_t elems = 3 * canvas_w * canvas_h;
    auto dst = device_alloc(ctx->device, elems * sizeof(float));
    run_preprocess(ctx, image, corners, cw.data(), 1, (int)canvas_w, (int)canvas_h, detector != 0,
                   static_cast<float*>(dst->ptr));
    HIP_OK(hipMemcpy(out_nchw, dst->ptr, elems * sizeof(float), hipMemcpyDeviceToHost));
  });
}

ppocr_status ppocr_hip_benchmark(ppocr_hip_model* model, const float* nchw, size_t len, size_t warmup, size_t runs,
                                 double* samples_ms) {
  return guarded([&] {
    if (!model || !samples_ms) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    if (runs == 0) raise(PPOCR_ERR_INVALID_INPUT, "runs must be positive");
    check_input(model, nchw, len);
    std::lock_guard<std::mutex> lock(model->ctx->mu);
    HIP_OK(hipSetDevice(model->ctx->device));
    ensure_arena(model->ctx, model->plan.arena_bytes);
    ensure_graph(model);
    upload_input(model, nchw, len);
    HIP_OK(hipStreamSynchronize(model->ctx->stream));
    for (size_t i = 0; i < warmup; ++i) run_graph(model);
    HIP_OK(hipStreamSynchronize(model->ctx->stream));
    for (size_t i = 0; i < runs; ++i) {
      auto t0 = std::chrono::steady_clock::now();
      run_graph(model);
      HIP_OK(hipStreamSynchronize(model->ctx->stream));
      auto t1 = std::chrono::steady_clock::now();
      samples_ms[i] = std::chrono::duration<double, std::milli>(t1 - t0).count();
    }
  });
}

ppocr_status ppocr_hip_benchmark_stream(ppocr_hip_model* model, const float* nchw, size_t len, size_t warmup,
                                        size_t runs, double* total_ms) {
  return guarded([&] {
    if (!model || !total_ms) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    if (runs == 0) raise(PPOCR_ERR_INVALID_INPUT, "runs must be positive");
    check_input(model, nchw, len);
    std::lock_guard<std::mutex> lock(model->ctx->mu);
    HIP_OK(hipSetDevice(model->ctx->device));
    ensure_arena(model->ctx, model->plan.arena_bytes);
    ensure_graph(model);
    upload_input(model, nchw, len);
    for (size_t i = 0; i < warmup; ++i) run_graph(model);
    HIP_OK(hipStreamSynchronize(model->ctx->stream));
    auto t0 = std::chrono::steady_clock::now();
    for (size_t i = 0; i < runs; ++i) run_graph(model);
    HIP_OK(hipStreamSynchronize(model->ctx->stream));
    auto t1 = std::chrono::steady_clock::now();
    *total_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
  });
}

ppocr_status ppocr_hip_profile(ppocr_hip_model* model, const float* nchw, size_t len, size_t runs,
                               ppocr_kernel_stat* stats, size_t cap, size_t* count) {
  return guarded([&] {
    if (!model || !count) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    if (runs == 0) raise(PPOCR_ERR_INVALID_INPUT, "runs must be positive");
    check_input(model, nchw, len);
    std::lock_guard<std::mutex> lock(model->ctx->mu);
    HIP_OK(hipSetDevice(model->ctx->device));
    ensure_arena(model->ctx, model->plan.arena_bytes);
    hipStream_t s = model->ctx->stream;
    upload_input(model, nchw, len);
    const auto& ops = model->plan.ops;
    std::vector<hipEvent_t> ev(ops.size() + 1);
    for (auto& e : ev) HIP_OK(hipEventCreate(&e));
    std::vector<double> total(ops.size(), 0.0);
    Exec ex = exec_of(model);
    // One untimed pass warms caches and code objects.
    for (const Op& op : ops) op.launch(ex, s);
    HIP_OK(hipStreamSynchronize(s));
    hipError_t err = hipSuccess;
    for (size_t r = 0; r < runs && err == hipSuccess; ++r) {
      for (size_t i = 0; i < ops.size(); ++i) {
        (void)hipEventRecord(ev[i], s);
        ops[i].launch(ex, s);
      }
      (void)hipEventRecord(ev[ops.size()], s);
      err = hipEventSynchronize(ev[ops.size()]);
      for (size_t i = 0; i < ops.size() && err == hipSuccess; ++i) {
        float ms = 0.0f;
        err = hipEventElapsedTime(&ms, ev[i], ev[i + 1]);
        total[i] += ms;
      }
    }
    for (auto& e : ev) (void)hipEventDestroy(e);
    HIP_OK(err);
    *count = ops.size();
    for (size_t i = 0; i < ops.size() && i < cap && stats; ++i) {
      ppocr_kernel_stat& st = stats[i];
      memset(&st, 0, sizeof st);
      strncpy(st.name, ops[i].name.c_str(), sizeof st.name - 1);
      strncpy(st.kernel, ops[i].kernel.c_str(), sizeof st.kernel - 1);
      st.avg_ms = total[i] / (double)runs;
      st.flops = ops[i].flops;
      st.bytes = ops[i].bytes;
      st.bound = ops[i].bound;
    }
  });
}

ppocr_status ppocr_hip_memory_report(const ppocr_hip_model* model, size_t* arena_bytes, size_t* unplanned_bytes,
                                     size_t* weight_bytes) {
  return guarded([&] {
    if (!model) raise(PPOCR_ERR_INVALID_INPUT, "model is null");
    if (arena_bytes) *arena_bytes = model->plan.arena_bytes;
    if (unplanned_bytes) *unplanned_bytes = model->plan.unplanned_bytes;
    if (weight_bytes) *weight_bytes = model->weights ? model->weights->bytes : 0;
  });
}

}  // extern "C"
