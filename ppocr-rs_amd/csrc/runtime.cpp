// Contexts, sessions and the C ABI (include/ppocr_hip.h).
//
// A context is one device, one stream and one activation arena shared by all
// of its models (the reference's shared workspace, src/gpu/runtime.rs:80-83,
// :1718-1730): the arena grows to the largest plan loaded on it.  A model's
// launch list is captured once into a hipGraph and replayed; the capture is
// redone whenever the arena had to move.
#include <chrono>
#include <cmath>
#include <cstdio>
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
  void* geo = nullptr;      // crop geometry of the synchronous image calls, grown on demand
  size_t geo_bytes = 0;
  void* db_scratch_ptr = nullptr;  // this device's static postprocess scratch (not owned)
  ~ppocr_hip_ctx() {
    (void)hipSetDevice(device);
    if (stream) (void)hipStreamSynchronize(stream);
    if (arena) (void)hipFree(arena);
    if (geo) (void)hipFree(geo);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

struct ppocr_hip_model {
  ppocr_hip_ctx* ctx = nullptr;
  ppocr::Plan plan;
  size_t in_shape[4] = {0, 0, 0, 0};
  // The plan (and its graph) covers `chunk` items; a batch of in_shape[0]
  // items runs as ceil(in_shape[0] / chunk) graph replays.  chunk < batch
  // only when one buffer of the whole-batch plan would pass the per-buffer
  // limit (kernels index a buffer with 32-bit offsets).
  size_t chunk = 0;
  size_t item_in = 0, item_out = 0;  // fp32 input / output elements per item
  std::vector<size_t> out_shape;     // whole-batch output shape
  std::shared_ptr<ppocr::DeviceBuffer> weights;
  size_t weight_blob_bytes = 0;
  std::string weights_path;
  int size = 0;
  hipGraphExec_t graph = nullptr;
  // The plan without its first op (the NCHW -> NHWC4 input conversion), for
  // inputs that device preprocessing writes as NHWC4 directly.
  hipGraphExec_t image_graph = nullptr;
  uint64_t graph_generation = UINT64_MAX;
  std::shared_ptr<ppocr::DeviceBuffer> db_work;  // postprocess work arrays, grown on demand
  ~ppocr_hip_model() {
    if (graph) (void)hipGraphExecDestroy(graph);
    if (image_graph) (void)hipGraphExecDestroy(image_graph);
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

void launch_all(ppocr_hip_model* m, hipStream_t s, size_t first = 0) {
  Exec ex = exec_of(m);
  for (size_t i = first; i < m->plan.ops.size(); ++i) m->plan.ops[i].launch(ex, s);
}

// Whether the plan starts with the NCHW -> NHWC4 input conversion, which
// device preprocessing can do itself.
bool direct_input(const ppocr_hip_model* m) { return !m->plan.ops.empty() && m->plan.ops[0].name == "input"; }

// Captures the launch list from op `first` on into an instantiated graph.
hipGraphExec_t capture(ppocr_hip_model* m, size_t first) {
  ppocr_hip_ctx* ctx = m->ctx;
  hipGraph_t graph = nullptr;
  HIP_OK(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
  launch_all(m, ctx->stream, first);
  hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    raise(PPOCR_ERR_GPU, std::string("graph capture failed: ") + hipGetErrorString(e));
  }
  hipGraphExec_t exec = nullptr;
  hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (ie != hipSuccess) raise(PPOCR_ERR_GPU, std::string("graph instantiate failed: ") + hipGetErrorString(ie));
  return exec;
}

// Captures the launch list into a graph (and the list without its input
// conversion into the image graph) if the arena moved since the last
// capture (caller holds ctx->mu and has sized the arena).
void ensure_graph(ppocr_hip_model* m) {
  ppocr_hip_ctx* ctx = m->ctx;
  if (m->graph && m->graph_generation == ctx->generation) return;
  for (hipGraphExec_t* g : {&m->graph, &m->image_graph})
    if (*g) {
      HIP_OK(hipGraphExecDestroy(*g));
      *g = nullptr;
    }
  // Queued work of other models may still be pending on the stream (the
  // engine's batch queue): let it drain so the capture starts from an idle stream.
  HIP_OK(hipStreamSynchronize(ctx->stream));
  m->graph = capture(m, 0);
  if (direct_input(m)) m->image_graph = capture(m, 1);
  m->graph_generation = ctx->generation;
}

size_t n_chunks(const ppocr_hip_model* m) { return (m->in_shape[0] + m->chunk - 1) / m->chunk; }
// Items of chunk c (the last one may be partial; the graph still runs a
// whole chunk, on the previous chunk's leftover inputs in the unused slots,
// whose outputs are not read).
size_t chunk_items(const ppocr_hip_model* m, size_t c) { return std::min(m->chunk, m->in_shape[0] - c * m->chunk); }
size_t output_elems(const ppocr_hip_model* m) { return m->item_out * m->in_shape[0]; }

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
// Device pointer of the plan's NHWC4 model input.
void* input_ptr(ppocr_hip_model* m) { return exec_of(m).ptr(m->plan.input); }

// Copies the NCHW input items of chunk c into the staging buffer.
void upload_chunk(ppocr_hip_model* m, const float* nchw, size_t c) {
  HIP_OK(hipMemcpyAsync(staging_ptr(m), nchw + c * m->chunk * m->item_in, chunk_items(m, c) * m->item_in * sizeof(float),
                        hipMemcpyHostToDevice, m->ctx->stream));
}

void run_graph(ppocr_hip_model* m) { HIP_OK(hipGraphLaunch(m->graph, m->ctx->stream)); }
// Runs the plan on an input that preprocess_chunk / enqueue_forward_image
// wrote: NHWC4 when the plan allows it (the image graph), else the staging
// planes (the whole graph).
void run_image_graph(ppocr_hip_model* m) {
  HIP_OK(hipGraphLaunch(m->image_graph ? m->image_graph : m->graph, m->ctx->stream));
}

void check_output_cap(ppocr_hip_model* m, const float* out, size_t cap) {
  const size_t n = output_elems(m);
  if (!out || cap < n)
    raise(PPOCR_ERR_INVALID_INPUT, "output capacity " + std::to_string(cap) + " is below " + std::to_string(n));
}

// Queues the download of chunk c's outputs into their place in `out`.
void download_chunk(ppocr_hip_model* m, float* out, size_t c) {
  HIP_OK(hipMemcpyAsync(out + c * m->chunk * m->item_out, output_ptr(m), chunk_items(m, c) * m->item_out * sizeof(float),
                        hipMemcpyDeviceToHost, m->ctx->stream));
}

// Waits for the queued downloads and rejects non-finite outputs
// (src/gpu/runtime.rs:2217-2219).
void finish_output(ppocr_hip_model* m, const float* out) {
  HIP_OK(hipStreamSynchronize(m->ctx->stream));
  const size_t n = output_elems(m);
  for (size_t i = 0; i < n; ++i)
    if (!std::isfinite(out[i])) raise(PPOCR_ERR_GPU, "model output contains non-finite values");
}

// Runs the whole batch from host NCHW input to host output.  The output of
// a chunk is downloaded before the next chunk's input overwrites staging (the
// stream orders the copies after the graph that reads and writes them).
void run_batch(ppocr_hip_model* m, const float* nchw, float* out) {
  for (size_t c = 0; c < n_chunks(m); ++c) {
    upload_chunk(m, nchw, c);
    run_graph(m);
    download_chunk(m, out, c);
  }
  finish_output(m, out);
}

// Largest buffer one plan may hold: every kernel addresses a buffer with
// 32-bit signed byte offsets.  PPOCR_HIP_MAX_BUFFER_BYTES lowers it (tests
// use it to exercise chunked batches at small shapes).
size_t max_buffer_bytes() {
  size_t limit = (size_t)INT32_MAX;
  if (const char* e = std::getenv("PPOCR_HIP_MAX_BUFFER_BYTES")) {
    const unsigned long long v = std::strtoull(e, nullptr, 10);
    if (v > 0 && v < limit) limit = (size_t)v;
  }
  return limit;
}

size_t largest_buffer(const Plan& plan) {
  size_t b = 0;
  for (const Buffer& buf : plan.bufs) b = std::max(b, buf.bytes);
  return b;
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
  auto build = [&](const size_t* shape) {
    return detector ? build_detector(st, size, shape, dt) : build_recognizer(st, size, shape, dt, greedy);
  };
  m->plan = build(nchw);
  m->chunk = nchw[0];
  m->out_shape = m->plan.output_shape;
  const size_t limit = max_buffer_bytes(), largest = largest_buffer(m->plan);
  if (largest > limit) {
    // Every buffer scales with the batch: plan the largest chunk that fits.
    const size_t per_item = (largest + nchw[0] - 1) / nchw[0];
    m->chunk = limit / per_item;
    if (m->chunk == 0)
      raise(PPOCR_ERR_INVALID_INPUT, "one input item needs a " + std::to_string(per_item) +
                                         "-byte activation buffer; the limit is " + std::to_string(limit) + " bytes");
    const size_t shape[4] = {m->chunk, nchw[1], nchw[2], nchw[3]};
    m->plan = build(shape);
    if (largest_buffer(m->plan) > limit)
      raise(PPOCR_ERR_INVALID_INPUT, "input too large for the per-buffer limit of " + std::to_string(limit) + " bytes");
  }
  m->item_in = nchw[1] * nchw[2] * nchw[3];
  m->item_out = m->plan.output_elems / m->chunk;
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
    HIP_OK(db_scratch(device, &ctx->db_scratch_ptr));
    *out = ctx.release();
  });
}

void ppocr_hip_destroy(ppocr_hip_ctx* ctx) { delete ctx; }

ppocr_status ppocr_hip_device_info(const ppocr_hip_ctx* ctx, ppocr_gpu_info* out) {
  return guarded([&] {
    if (!ctx || !out) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    hipDeviceProp_t prop{};
    HIP_OK(hipGetDeviceProperties(&prop, ctx->device));
    ppocr_gpu_info info{};
    snprintf(info.name, sizeof info.name, "%.255s", prop.name);
    snprintf(info.backend, sizeof info.backend, "HIP");
    snprintf(info.arch, sizeof info.arch, "%.63s", prop.gcnArchName);
    info.device = ctx->device;
    info.integrated = prop.integrated ? 1 : 0;
    info.compute_units = prop.multiProcessorCount;
    info.wavefront_size = prop.warpSize;
    info.total_memory = prop.totalGlobalMem;
    *out = info;
  });
}

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
    *rank = model->out_shape.size();
    for (size_t i = 0; i < 4; ++i) shape[i] = i < *rank ? model->out_shape[i] : 0;
  });
}

ppocr_status ppocr_hip_forward(ppocr_hip_model* model, const float* nchw, size_t len, float* out, size_t out_cap) {
  return guarded([&] {
    if (!model) raise(PPOCR_ERR_INVALID_INPUT, "model is null");
    check_input(model, nchw, len);
    check_output_cap(model, out, out_cap);
    std::lock_guard<std::mutex> lock(model->ctx->mu);
    HIP_OK(hipSetDevice(model->ctx->device));
    ensure_arena(model->ctx, model->plan.arena_bytes);
    ensure_graph(model);
    run_batch(model, nchw, out);
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

// Enqueues the device preprocessing of `n` geometries into `dst` (fp32 NCHW
// planes) on the context stream; `geo` is the geometry table in device
// memory: corners [n][8] floats, then content widths [n] ints.  Caller holds
// ctx->mu.
void enqueue_preprocess(ppocr_hip_ctx* ctx, const ppocr_hip_image* image, const void* geo, int n, int cw, int ch,
                        bool detector, float* dst, void* nhwc4 = nullptr, int dt = DT_F32) {
  static const float det_mean[3] = {0.485f, 0.456f, 0.406f}, det_std[3] = {0.229f, 0.224f, 0.225f};
  static const float rec_mean[3] = {0.5f, 0.5f, 0.5f}, rec_std[3] = {0.5f, 0.5f, 0.5f};
  const float* mean = detector ? det_mean : rec_mean;
  const float* stdv = detector ? det_std : rec_std;
  PreParams p{};
  p.rgb = static_cast<const uint32_t*>(image->pixels->ptr);
  p.sw = (int)image->width;
  p.sh = (int)image->height;
  p.corners = static_cast<const float*>(geo);
  p.content_w = reinterpret_cast<const int*>(static_cast<const char*>(geo) + (size_t)n * 8 * sizeof(float));
  p.N = n;
  p.cw = cw;
  p.ch = ch;
  for (int c = 0; c < 3; ++c) {
    p.scale[c] = 1.0f / (255.0f * stdv[c]);
    p.bias[c] = -mean[c] / stdv[c];
  }
  p.out = dst;
  p.nhwc4 = nhwc4;
  p.dt = dt;
  launch_preprocess(p, ctx->stream);
  HIP_OK(hipGetLastError());
}

void pack_geometry(char* dst, const float* corners, const int* content_w, size_t n) {
  memcpy(dst, corners, n * 8 * sizeof(float));
  memcpy(dst + n * 8 * sizeof(float), content_w, n * sizeof(int));
}

// Queues the upload of items [first, first + n) of a packed geometry table
// of `total` items (corners, then widths) as an n-item table at `geo`.
void upload_geometry_slice(ppocr_hip_ctx* ctx, const char* packet, size_t total, size_t first, size_t n) {
  char* geo = static_cast<char*>(ctx->geo);
  HIP_OK(hipMemcpyAsync(geo, packet + first * 8 * sizeof(float), n * 8 * sizeof(float), hipMemcpyHostToDevice,
                        ctx->stream));
  HIP_OK(hipMemcpyAsync(geo + n * 8 * sizeof(float), packet + total * 8 * sizeof(float) + first * sizeof(int),
                        n * sizeof(int), hipMemcpyHostToDevice, ctx->stream));
}

// Sizes the context's device geometry buffer to at least `bytes`; a move
// waits for the queued work that may still read the old one.  Caller holds
// ctx->mu.
void ensure_geometry(ppocr_hip_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->geo_bytes) return;
  HIP_OK(hipStreamSynchronize(ctx->stream));
  if (ctx->geo) HIP_OK(hipFree(ctx->geo));
  ctx->geo = nullptr;
  ctx->geo_bytes = 0;
  HIP_OK(hipMalloc(&ctx->geo, bytes));
  ctx->geo_bytes = bytes;
}

// Runs the device preprocessing of `n` geometries into `dst` and waits for
// it: the geometry goes through the context's geometry buffer, which the
// next call may overwrite.  Caller holds ctx->mu.
void run_preprocess(ppocr_hip_ctx* ctx, const ppocr_hip_image* image, const float* corners, const int* content_w,
                    int n, int cw, int ch, bool detector, float* dst, void* nhwc4 = nullptr, int dt = DT_F32) {
  const size_t bytes = packet_bytes((size_t)n);
  ensure_geometry(ctx, bytes);
  std::vector<char> host(bytes);
  pack_geometry(host.data(), corners, content_w, (size_t)n);
  HIP_OK(hipMemcpyAsync(ctx->geo, host.data(), bytes, hipMemcpyHostToDevice, ctx->stream));
  enqueue_preprocess(ctx, image, ctx->geo, n, cw, ch, detector, dst, nhwc4, dt);
  // `host` is pageable and goes out of scope here.
  HIP_OK(hipStreamSynchronize(ctx->stream));
}

// Preprocesses chunk c of a model's image batch and waits for it: into the
// NHWC4 model input when the plan starts with the input conversion (run
// the image graph next), else into the staging planes.  Caller holds
// ctx->mu and has run ensure_graph.
void preprocess_chunk(ppocr_hip_model* m, const ppocr_hip_image* image, const float* corners, const int* content_w,
                      size_t c) {
  const size_t first = c * m->chunk;
  const bool direct = m->image_graph != nullptr;
  run_preprocess(m->ctx, image, corners + first * 8, content_w + first, (int)chunk_items(m, c), (int)m->in_shape[3],
                 (int)m->in_shape[2], m->plan.detector, direct ? nullptr : staging_ptr(m),
                 direct ? input_ptr(m) : nullptr, m->plan.input.dt);
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

// Geometry packet of `n` crops: corners [n][8] floats, then content widths
// [n] ints.
size_t packet_bytes(size_t n) { return n * 8 * sizeof(float) + n * sizeof(int); }

void enqueue_forward_image(ppocr_hip_model* model, const ppocr_hip_image* image, const float* corners,
                           const size_t* content_w, size_t n, char* packet, float* out, size_t out_cap) {
  if (!model || !image || !packet || !out) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
  if (image->ctx != model->ctx) raise(PPOCR_ERR_INVALID_INPUT, "image and model belong to different contexts");
  if (n != model->in_shape[0])
    raise(PPOCR_ERR_INVALID_INPUT, "geometry count " + std::to_string(n) + " differs from the planned batch");
  check_output_cap(model, out, out_cap);
  check_corners(corners, n);
  std::vector<int> cw = content_widths(content_w, n, model->in_shape[3]);
  pack_geometry(packet, corners, cw.data(), n);
  ppocr_hip_ctx* ctx = model->ctx;
  std::lock_guard<std::mutex> lock(ctx->mu);
  HIP_OK(hipSetDevice(ctx->device));
  ensure_arena(ctx, model->plan.arena_bytes);
  ensure_graph(model);
  // One geometry buffer serves every queued batch and chunk: each upload is
  // ordered after the previous preprocess on the stream.
  ensure_geometry(ctx, packet_bytes(model->chunk));
  for (size_t c = 0; c < n_chunks(model); ++c) {
    const size_t items = chunk_items(model, c);
    upload_geometry_slice(ctx, packet, n, c * model->chunk, items);
    const bool direct = model->image_graph != nullptr;
    enqueue_preprocess(ctx, image, ctx->geo, (int)items, (int)model->in_shape[3], (int)model->in_shape[2],
                       model->plan.detector, direct ? nullptr : staging_ptr(model),
                       direct ? input_ptr(model) : nullptr, model->plan.input.dt);
    run_image_graph(model);
    download_chunk(model, out, c);
  }
}

void sync_context(ppocr_hip_ctx* ctx) {
  HIP_OK(hipSetDevice(ctx->device));
  HIP_OK(hipStreamSynchronize(ctx->stream));
}

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
    check_output_cap(model, out, out_cap);
    std::lock_guard<std::mutex> lock(model->ctx->mu);
    HIP_OK(hipSetDevice(model->ctx->device));
    ensure_arena(model->ctx, model->plan.arena_bytes);
    ensure_graph(model);
    // Preprocess straight into the model input the image graph starts from.
    for (size_t c = 0; c < n_chunks(model); ++c) {
      preprocess_chunk(model, image, corners, cw.data(), c);
      run_image_graph(model);
      download_chunk(model, out, c);
    }
    finish_output(model, out);
  });
}

ppocr_status ppocr_hip_preprocess(ppocr_hip_ctx* ctx, const ppocr_hip_image* image, const float corners[8],
                                  size_t canvas_w, size_t canvas_h, size_t content_width, int detector,
                                  float* out_nchw) {
  return guarded([&] {
    if (!ctx || !image || !out_nchw) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    if (canvas_w == 0 || canvas_h == 0 || canvas_w > (1u << 18) || canvas_h > (1u << 15))
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
    // Device-only timing, like benchmark_nchw: the input is staged once
    // (the first chunk's items) and each run replays the graph once per chunk.
    upload_chunk(model, nchw, 0);
    HIP_OK(hipStreamSynchronize(model->ctx->stream));
    const size_t chunks = n_chunks(model);
    for (size_t i = 0; i < warmup; ++i)
      for (size_t c = 0; c < chunks; ++c) run_graph(model);
    HIP_OK(hipStreamSynchronize(model->ctx->stream));
    for (size_t i = 0; i < runs; ++i) {
      auto t0 = std::chrono::steady_clock::now();
      for (size_t c = 0; c < chunks; ++c) run_graph(model);
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
    upload_chunk(model, nchw, 0);
    const size_t chunks = n_chunks(model);
    for (size_t i = 0; i < warmup * chunks; ++i) run_graph(model);
    HIP_OK(hipStreamSynchronize(model->ctx->stream));
    auto t0 = std::chrono::steady_clock::now();
    for (size_t i = 0; i < runs * chunks; ++i) run_graph(model);
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
    upload_chunk(model, nchw, 0);
    const size_t chunks = n_chunks(model);
    const auto& ops = model->plan.ops;
    std::vector<hipEvent_t> ev(ops.size() + 1);
    for (auto& e : ev) HIP_OK(hipEventCreate(&e));
    std::vector<double> total(ops.size(), 0.0);
    Exec ex = exec_of(model);
    // One untimed pass warms caches and code objects.
    for (const Op& op : ops) op.launch(ex, s);
    HIP_OK(hipStreamSynchronize(s));
    hipError_t err = hipSuccess;
    // A run covers the whole batch: every op once per chunk.
    for (size_t r = 0; r < runs * chunks && err == hipSuccess; ++r) {
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

// ------------------------------------------------------------ DB postprocess
namespace ppocr {

ppocr_db_options db_options(const ppocr_db_options* o) {
  ppocr_db_options v;
  ppocr_db_default_options(&v);
  if (o) v = *o;
  // DetectorPostprocessOptions::validate (src/ocr.rs:250-268).
  auto prob = [](float x) { return std::isfinite(x) && x >= 0.0f && x <= 1.0f; };
  if (!prob(v.binary_threshold)) raise(PPOCR_ERR_INVALID_INPUT, "detector binary threshold must be a finite value between zero and one");
  if (!prob(v.box_threshold)) raise(PPOCR_ERR_INVALID_INPUT, "detector box threshold must be a finite value between zero and one");
  if (v.min_area == 0) raise(PPOCR_ERR_INVALID_INPUT, "detector minimum area must be at least one pixel");
  if (v.max_boxes == 0) raise(PPOCR_ERR_INVALID_INPUT, "detector maximum box count must be at least one");
  if (!std::isfinite(v.unclip_ratio) || v.unclip_ratio <= 0.0f)
    raise(PPOCR_ERR_INVALID_INPUT, "detector unclip ratio must be a finite value greater than zero");
  return v;
}

namespace {

struct HostDetection {
  ppocr_detection det;
  int image;
  int root;
  float cx, cy;  // polygon_center, computed once for the sorts
};

// polygon_center (src/ocr.rs:1133-1138) in f32.
void polygon_center(const ppocr_detection& d, float* cx, float* cy) {
  float sx = 0.0f, sy = 0.0f;
  for (int k = 0; k < 4; ++k) sx += d.polygon[2 * k];
  for (int k = 0; k < 4; ++k) sy += d.polygon[2 * k + 1];
  *cx = sx / 4.0f;
  *cy = sy / 4.0f;
}

// A key whose unsigned order is f32::total_cmp's order (negative values
// below -0, below +0, below positive values).
uint32_t total_key(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Byte offsets of the postprocess work arrays of N maps of H x W in one
// work buffer (256-byte aligned), and its size.
struct DbLayout {
  size_t label, slot, counters, tables, count, root, keep, mom, geom, ext, out, bytes;
  long max_comp;
};

DbLayout db_layout(int N, int H, int W) {
  DbLayout l;
  const size_t total = (size_t)N * H * W;
  // At most one component per 2x2 pixel block: two pixels of one block are
  // 8-neighbours, so they cannot start different components.
  l.max_comp = (long)N * ((H + 1) / 2) * ((W + 1) / 2);
  const size_t mc = (size_t)l.max_comp;
  size_t off = 0;
  auto carve = [&](size_t bytes) {
    size_t at = off;
    off += (bytes + 255) / 256 * 256;
    return at;
  };
  l.label = carve(4 * total);
  l.slot = carve(4 * total);
  l.counters = carve(12);
  l.tables = carve(4 * 6 * (size_t)N);
  l.count = carve(4 * mc);
  l.root = carve(4 * mc);
  l.keep = carve(4 * mc);
  l.mom = carve(48 * mc);
  l.geom = carve(32 * mc);
  l.ext = carve(16 * mc);
  l.out = carve(48 * mc);
  l.bytes = off;
  return l;
}

// Grows a model's or call's postprocess work buffer to `bytes`.
// PPOCR_HIP_DB_PROFILE set: each postprocess run prints one JSON line to
// stderr with the wall time of its host steps and the HIP-event time of each
// of its kernels (ms), like the reference's PPOCR_GPU_PROFILE dispatch
// profile (src/gpu/runtime.rs:1815-1817).
class DbProfile {
 public:
  DbProfile() : on_(std::getenv("PPOCR_HIP_DB_PROFILE") != nullptr) {
    if (!on_) return;
    for (hipEvent_t& e : ev_) HIP_OK(hipEventCreate(&e));
    last_ = std::chrono::steady_clock::now();
  }
  ~DbProfile() {
    if (on_)
      for (hipEvent_t e : ev_) (void)hipEventDestroy(e);
  }
  hipEvent_t* marks() { return on_ ? ev_ : nullptr; }
  void step(const char* name) {
    if (!on_) return;
    const auto now = std::chrono::steady_clock::now();
    steps_.push_back({name, std::chrono::duration<double, std::milli>(now - last_).count()});
    last_ = now;
  }
  void report(int detections, int n, int h, int w) {
    if (!on_) return;
    std::string line = "{\"db_profile\": {\"maps\": [" + std::to_string(n) + ", " + std::to_string(h) + ", " +
                       std::to_string(w) + "], \"components_emitted\": " + std::to_string(detections) +
                       ", \"host_ms\": {";
    for (size_t i = 0; i < steps_.size(); ++i)
      line += (i ? ", \"" : "\"") + steps_[i].first + "\": " + std::to_string(steps_[i].second);
    line += "}, \"kernel_ms\": {";
    for (int i = 0; i < kDbKernels; ++i) {
      float ms = 0.0f;
      HIP_OK(hipEventElapsedTime(&ms, ev_[i], ev_[i + 1]));
      line += (i ? ", \"" : "\"") + std::string(kDbKernelNames[i]) + "\": " + std::to_string(ms);
    }
    line += "}}}\n";
    fputs(line.c_str(), stderr);
  }

 private:
  bool on_;
  hipEvent_t ev_[kDbKernels + 1] = {};
  std::chrono::steady_clock::time_point last_;
  std::vector<std::pair<std::string, double>> steps_;
};

char* db_work(ppocr_hip_ctx* ctx, std::shared_ptr<DeviceBuffer>& work, size_t bytes) {
  if (!work || work->bytes < bytes) work = device_alloc(ctx->device, bytes);
  return static_cast<char*>(work->ptr);
}

// Runs the device postprocess over N maps already in device memory and
// returns the per-image sorted, truncated detections.  `base` holds at least
// db_layout(N, H, W).bytes of work space.  Caller holds ctx->mu.
std::vector<std::vector<HostDetection>> run_db(ppocr_hip_ctx* ctx, const float* prob, int N, int H, int W,
                                               const ppocr_detector_transform* tr, const ppocr_db_options& o,
                                               char* base, ppocr_status non_finite_status) {
  if (!tr) raise(PPOCR_ERR_INVALID_INPUT, "transforms pointer is null");
  const long total = (long)N * H * W;
  if (total >= (long)INT32_MAX) raise(PPOCR_ERR_INVALID_INPUT, "probability maps too large for the postprocess");
  const DbLayout L = db_layout(N, H, W);
  DbProfile prof;
  std::vector<int> tables(6 * (size_t)N);
  for (int n = 0; n < N; ++n) {
    const ppocr_detector_transform& t = tr[n];
    if (!t.source_width || !t.source_height || !t.content_width || !t.content_height)
      raise(PPOCR_ERR_INVALID_INPUT, "detector transform dimensions must be non-zero");
    tables[2 * n] = (int)std::min<uint32_t>(t.content_width, (uint32_t)W);
    tables[2 * n + 1] = (int)std::min<uint32_t>(t.content_height, (uint32_t)H);
    tables[2 * N + 2 * n] = (int)std::min<uint32_t>(t.source_width, INT32_MAX);
    tables[2 * N + 2 * n + 1] = (int)std::min<uint32_t>(t.source_height, INT32_MAX);
    tables[4 * N + 2 * n] = (int)std::min<uint32_t>(t.content_width, INT32_MAX);
    tables[4 * N + 2 * n + 1] = (int)std::min<uint32_t>(t.content_height, INT32_MAX);
  }
  HIP_OK(hipMemcpyAsync(base + L.tables, tables.data(), 4 * tables.size(), hipMemcpyHostToDevice, ctx->stream));
  prof.step("tables_h2d");
  DbParams p{};
  p.prob = prob;
  p.N = N, p.H = H, p.W = W;
  p.total = total;
  p.content = reinterpret_cast<const int*>(base + L.tables);
  p.source = p.content + 2 * N;
  p.content_scale = p.content + 4 * N;
  p.threshold = o.binary_threshold;
  p.box_threshold = o.box_threshold;
  p.unclip = o.unclip_ratio;
  p.min_area = (int)std::min<size_t>(o.min_area, (size_t)INT32_MAX);
  p.max_comp = (int)L.max_comp;
  p.label = reinterpret_cast<int*>(base + L.label);
  p.slot = reinterpret_cast<int*>(base + L.slot);
  p.counters = reinterpret_cast<int*>(base + L.counters);
  p.count = reinterpret_cast<int*>(base + L.count);
  p.root = reinterpret_cast<int*>(base + L.root);
  p.keep = reinterpret_cast<int*>(base + L.keep);
  p.moments = reinterpret_cast<double*>(base + L.mom);
  p.geom = reinterpret_cast<float*>(base + L.geom);
  p.extent = reinterpret_cast<int*>(base + L.ext);
  p.out = reinterpret_cast<float*>(base + L.out);
  launch_db_postprocess(p, ctx->stream, prof.marks());
  HIP_OK(hipGetLastError());
  prof.step("launch");
  // The counters and a first block of records come back in one round trip;
  // more records (a page with over kDbFirstRecords components) in a second.
  constexpr int kDbFirstRecords = 1024;
  const int first = (int)std::min<long>(kDbFirstRecords, p.max_comp);
  int counters[3] = {0, 0, 0};
  std::vector<float> rec(12 * (size_t)first);
  HIP_OK(hipMemcpyAsync(counters, p.counters, sizeof counters, hipMemcpyDeviceToHost, ctx->stream));
  HIP_OK(hipMemcpyAsync(rec.data(), p.out, rec.size() * 4, hipMemcpyDeviceToHost, ctx->stream));
  HIP_OK(hipStreamSynchronize(ctx->stream));
  prof.step("kernels_and_first_records_d2h");
  // src/ocr.rs:731-733
  if (counters[2]) raise(non_finite_status, "detector output contains non-finite values");
  const int n_det = std::max(0, std::min(counters[1], p.max_comp));
  if (n_det > first) {
    rec.resize(12 * (size_t)n_det);
    HIP_OK(hipMemcpyAsync(rec.data() + 12 * (size_t)first, p.out + 12 * (size_t)first,
                          12 * sizeof(float) * (size_t)(n_det - first), hipMemcpyDeviceToHost, ctx->stream));
    HIP_OK(hipStreamSynchronize(ctx->stream));
  }
  prof.step("more_records_d2h");
  // sort_detections, and the max_boxes cut by score (src/ocr.rs:775-788):
  // the kept detections are the first max_boxes under (score descending,
  // centre y, centre x, raster order), selected in linear time from packed
  // keys, and only those are sorted into (centre y, centre x, score, raster
  // order) and built.  The keys order as f32::total_cmp does.
  struct Key {
    uint64_t hi, lo;
    uint32_t i;
  };
  auto before = [](const Key& a, const Key& b) { return a.hi != b.hi ? a.hi < b.hi : a.lo < b.lo; };
  std::vector<std::vector<Key>> keys(N);
  std::vector<float> cx(n_det), cy(n_det);
  for (int i = 0; i < n_det; ++i) {
    const float* r = rec.data() + 12 * (size_t)i;
    int image;
    memcpy(&image, r + 9, 4);
    if (image < 0 || image >= N) raise(PPOCR_ERR_GPU, "postprocess produced an invalid image index");
    ppocr_detection d;
    memcpy(d.polygon, r, 8 * sizeof(float));
    polygon_center(d, &cx[i], &cy[i]);
    keys[image].push_back({0, 0, (uint32_t)i});
  }
  auto root_of = [&](uint32_t i) {
    int root;
    memcpy(&root, rec.data() + 12 * (size_t)i + 10, 4);
    return (uint32_t)root;
  };
  auto score_of = [&](uint32_t i) { return rec[12 * (size_t)i + 8]; };
  std::vector<std::vector<HostDetection>> per(N);
  for (int n = 0; n < N; ++n) {
    std::vector<Key>& k = keys[n];
    if (k.size() > o.max_boxes) {
      for (Key& e : k) {
        e.hi = ((uint64_t)~total_key(score_of(e.i)) << 32) | total_key(cy[e.i]);
        e.lo = ((uint64_t)total_key(cx[e.i]) << 32) | root_of(e.i);
      }
      std::nth_element(k.begin(), k.begin() + (long)o.max_boxes, k.end(), before);
      k.resize(o.max_boxes);
    }
    for (Key& e : k) {
      e.hi = ((uint64_t)total_key(cy[e.i]) << 32) | total_key(cx[e.i]);
      e.lo = ((uint64_t)total_key(score_of(e.i)) << 32) | root_of(e.i);
    }
    std::sort(k.begin(), k.end(), before);
    per[n].reserve(k.size());
    for (const Key& e : k) {
      HostDetection d;
      memcpy(d.det.polygon, rec.data() + 12 * (size_t)e.i, 8 * sizeof(float));
      d.det.score = score_of(e.i);
      d.image = n;
      d.root = (int)root_of(e.i);
      d.cx = cx[e.i];
      d.cy = cy[e.i];
      per[n].push_back(d);
    }
  }
  prof.step("host_sort");
  prof.report(n_det, N, H, W);
  return per;
}

void write_detections(const std::vector<std::vector<HostDetection>>& per, ppocr_detection* out, size_t cap,
                      size_t* counts, size_t* total) {
  size_t k = 0;
  for (size_t n = 0; n < per.size(); ++n) {
    if (counts) counts[n] = per[n].size();
    for (const HostDetection& d : per[n]) {
      if (out && k < cap) out[k] = d.det;
      ++k;
    }
  }
  if (total) *total = k;
}

}  // namespace
}  // namespace ppocr

extern "C" {

void ppocr_db_default_options(ppocr_db_options* o) {
  if (!o) return;
  o->binary_threshold = 0.2f;
  o->box_threshold = 0.4f;
  o->min_area = 3;
  o->unclip_ratio = 1.4f;
  o->max_boxes = 1000;
}

ppocr_status ppocr_hip_db_postprocess(ppocr_hip_ctx* ctx, const float* prob, size_t n, size_t height, size_t width,
                                      const ppocr_detector_transform* transforms, const ppocr_db_options* options,
                                      ppocr_detection* out, size_t cap, size_t* counts, size_t* total) {
  return guarded([&] {
    if (!ctx || !prob) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    if (n == 0 || height == 0 || width == 0) raise(PPOCR_ERR_INVALID_INPUT, "probability maps must be non-empty");
    if (n * height * width >= (size_t)INT32_MAX)
      raise(PPOCR_ERR_INVALID_INPUT, "probability maps too large for the postprocess");
    const ppocr_db_options o = db_options(options);
    const size_t elems = n * height * width;
    // Non-finite map values are found by the device pass (counters[2]) and
    // reported as invalid input for caller-supplied maps.
    std::lock_guard<std::mutex> lock(ctx->mu);
    HIP_OK(hipSetDevice(ctx->device));
    auto maps = device_alloc(ctx->device, elems * sizeof(float));
    HIP_OK(hipMemcpyAsync(maps->ptr, prob, elems * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
    std::shared_ptr<DeviceBuffer> work;
    char* base = db_work(ctx, work, db_layout((int)n, (int)height, (int)width).bytes);
    auto per = run_db(ctx, static_cast<const float*>(maps->ptr), (int)n, (int)height, (int)width, transforms, o, base,
                      PPOCR_ERR_INVALID_INPUT);
    write_detections(per, out, cap, counts, total);
  });
}

// The no-allocation variant: the maps are staged, and the work arrays laid
// out, in the library's static device scratch (db_scratch), whose address
// was looked up for the context's device by ppocr_hip_create.
ppocr_status ppocr_hip_db_postprocess_static(ppocr_hip_ctx* ctx, const float* prob, size_t n, size_t height,
                                             size_t width, const ppocr_detector_transform* transforms,
                                             const ppocr_db_options* options, ppocr_detection* out, size_t cap,
                                             size_t* counts, size_t* total) {
  return guarded([&] {
    if (!ctx || !prob) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    if (n == 0 || height == 0 || width == 0) raise(PPOCR_ERR_INVALID_INPUT, "probability maps must be non-empty");
    if (n * height * width >= (size_t)INT32_MAX)
      raise(PPOCR_ERR_INVALID_INPUT, "probability maps too large for the postprocess");
    const ppocr_db_options o = db_options(options);
    const size_t elems = n * height * width;
    const size_t map_bytes = (elems * sizeof(float) + 255) / 256 * 256;
    const size_t need = map_bytes + db_layout((int)n, (int)height, (int)width).bytes;
    if (need > db_scratch_bytes())
      raise(PPOCR_ERR_INVALID_INPUT, "maps need " + std::to_string(need) + " bytes of postprocess scratch; the static "
                                     "scratch holds " + std::to_string(db_scratch_bytes()) + " bytes");
    std::lock_guard<std::mutex> lock(ctx->mu);
    // Every context on this device shares its scratch: hold the device's
    // scratch lock from staging the maps until the detections are read back.
    std::mutex* device_mu = db_scratch_mutex(ctx->device);
    if (!device_mu) raise(PPOCR_ERR_GPU, "postprocess scratch unavailable for this device index");
    std::lock_guard<std::mutex> scratch_lock(*device_mu);
    HIP_OK(hipSetDevice(ctx->device));
    char* base = static_cast<char*>(ctx->db_scratch_ptr);
    if (!base) raise(PPOCR_ERR_GPU, "postprocess scratch address unknown for this device");
    HIP_OK(hipMemcpyAsync(base, prob, elems * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
    auto per = run_db(ctx, reinterpret_cast<const float*>(base), (int)n, (int)height, (int)width, transforms, o,
                      base + map_bytes, PPOCR_ERR_INVALID_INPUT);
    write_detections(per, out, cap, counts, total);
  });
}

ppocr_status ppocr_hip_detect(ppocr_hip_model* model, const float* nchw, size_t len,
                              const ppocr_detector_transform* transforms, const ppocr_db_options* options,
                              ppocr_detection* out, size_t cap, size_t* counts, size_t* total) {
  return guarded([&] {
    if (!model) raise(PPOCR_ERR_INVALID_INPUT, "model is null");
    if (!model->plan.detector) raise(PPOCR_ERR_INVALID_INPUT, "detection needs a detector model");
    const ppocr_db_options o = db_options(options);
    check_input(model, nchw, len);
    if (!transforms) raise(PPOCR_ERR_INVALID_INPUT, "transforms pointer is null");
    std::lock_guard<std::mutex> lock(model->ctx->mu);
    HIP_OK(hipSetDevice(model->ctx->device));
    ensure_arena(model->ctx, model->plan.arena_bytes);
    ensure_graph(model);
    const auto& s = model->plan.output_shape;
    std::vector<std::vector<HostDetection>> per;
    for (size_t c = 0; c < n_chunks(model); ++c) {
      upload_chunk(model, nchw, c);
      run_graph(model);
      const int items = (int)chunk_items(model, c);
      char* base = db_work(model->ctx, model->db_work, db_layout(items, (int)s[2], (int)s[3]).bytes);
      auto part = run_db(model->ctx, output_ptr(model), items, (int)s[2], (int)s[3], transforms + c * model->chunk, o,
                         base, PPOCR_ERR_GPU);
      for (auto& v : part) per.push_back(std::move(v));
    }
    write_detections(per, out, cap, counts, total);
  });
}

ppocr_status ppocr_hip_detect_image(ppocr_hip_model* model, const ppocr_hip_image* image, const float* corners,
                                    size_t n, const ppocr_detector_transform* transforms,
                                    const ppocr_db_options* options, ppocr_detection* out, size_t cap,
                                    size_t* counts, size_t* total) {
  return guarded([&] {
    if (!model || !image) raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    if (!model->plan.detector) raise(PPOCR_ERR_INVALID_INPUT, "detection needs a detector model");
    if (image->ctx != model->ctx) raise(PPOCR_ERR_INVALID_INPUT, "image and model belong to different contexts");
    if (n != model->in_shape[0])
      raise(PPOCR_ERR_INVALID_INPUT, "geometry count " + std::to_string(n) + " differs from the planned batch");
    check_corners(corners, n);
    const ppocr_db_options o = db_options(options);
    std::vector<int> cw = content_widths(nullptr, n, model->in_shape[3]);
    if (!transforms) raise(PPOCR_ERR_INVALID_INPUT, "transforms pointer is null");
    std::lock_guard<std::mutex> lock(model->ctx->mu);
    HIP_OK(hipSetDevice(model->ctx->device));
    ensure_arena(model->ctx, model->plan.arena_bytes);
    ensure_graph(model);
    const auto& s = model->plan.output_shape;
    std::vector<std::vector<HostDetection>> per;
    for (size_t c = 0; c < n_chunks(model); ++c) {
      preprocess_chunk(model, image, corners, cw.data(), c);
      run_image_graph(model);
      const int items = (int)chunk_items(model, c);
      char* base = db_work(model->ctx, model->db_work, db_layout(items, (int)s[2], (int)s[3]).bytes);
      auto part = run_db(model->ctx, output_ptr(model), items, (int)s[2], (int)s[3], transforms + c * model->chunk, o,
                         base, PPOCR_ERR_GPU);
      for (auto& v : part) per.push_back(std::move(v));
    }
    write_detections(per, out, cap, counts, total);
  });
}

}  // extern "C"
