// End-to-end OCR engine over the HIP backend: the GPU arm of the reference's
// OcrEngine (src/ocr.rs:354-600) with its session caches (GpuOcrRuntime,
// src/ocr.rs:608-689).
//
// recognize() follows recognize_with (src/ocr.rs:524-600):
//   detector input plan -> detector on the device image -> device DB
//   postprocess -> crops ordered by aspect ratio -> batches of 6 with a
//   shared canvas width -> recognizer on device-rectified crops -> greedy
//   CTC.
// Departures, all on the device side of the boundary: the detector's
// probability map never leaves HBM (postprocess on the device); every crop
// of a recognizer batch is rectified on the device (the reference prepares
// them on the host, src/ocr.rs:653); and, by default, the recognizer runs
// with the classifier fused with per-step greedy decoding, so only (class,
// probability) per time step is copied back.
//
// Caches: two detector plans and four recognizer plans, keyed by input
// shape, oldest evicted first (src/ocr.rs:27-30, :614-640, :655-685); every
// recognizer plan shares one copy of the device weights.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <numeric>
#include <vector>

#include "runtime.h"

namespace {

constexpr size_t DETECTOR_CACHE_LIMIT = 2;    // src/ocr.rs:28
constexpr size_t RECOGNIZER_CACHE_LIMIT = 4;  // src/ocr.rs:30
constexpr size_t RECOGNIZER_BATCH_SIZE = 6;   // src/ocr.rs:22

void check(ppocr_status s) {
  if (s != PPOCR_OK) ppocr::raise(s, ppocr_hip_last_error());
}

struct ModelHandle {
  ppocr_hip_model* m = nullptr;
  explicit ModelHandle(ppocr_hip_model* p) : m(p) {}
  ModelHandle(const ModelHandle&) = delete;
  ModelHandle& operator=(const ModelHandle&) = delete;
  ~ModelHandle() { ppocr_hip_model_free(m); }
};

struct ImageHandle {
  ppocr_hip_image* p = nullptr;
  ~ImageHandle() { ppocr_hip_image_free(p); }
};

struct Cached {
  size_t shape[4];
  std::unique_ptr<ModelHandle> model;
};

float edge(const float* p, int a, int b) {
  const float dx = p[2 * a] - p[2 * b], dy = p[2 * a + 1] - p[2 * b + 1];
  const float sx = dx * dx;
  const float sy = dy * dy;
  return std::sqrt(sx + sy);
}

// polygon_aspect_ratio (src/ocr.rs:1139-1143).
float aspect_ratio(const float* p) {
  const float w = std::max(edge(p, 0, 1), edge(p, 3, 2));
  const float h = std::max(edge(p, 0, 3), edge(p, 1, 2));
  return w / std::max(h, 1.1920929e-7f);
}

// f32::total_cmp on finite values.
bool total_less(float a, float b) {
  if (a != b) return a < b;
  return std::signbit(a) && !std::signbit(b);
}

// Pinned host staging of the queued recognizer batches of one page: each
// batch's geometry packet (read by its upload) and its per-step (class,
// probability) pairs (written by its download), 256-byte aligned slices.
struct PinnedStage {
  char* base = nullptr;
  size_t bytes = 0, used = 0;
  PinnedStage() = default;
  PinnedStage(const PinnedStage&) = delete;
  PinnedStage& operator=(const PinnedStage&) = delete;
  ~PinnedStage() {
    if (base) (void)hipHostFree(base);
  }
  static size_t round(size_t n) { return (n + 255) / 256 * 256; }
  char* take(size_t n) {
    n = round(n);
    if (used + n > bytes) return nullptr;
    char* p = base + used;
    used += n;
    return p;
  }
  // Replaces the area (nothing may be queued on it).
  void reserve(size_t n) {
    if (base) HIP_OK(hipHostFree(base));
    base = nullptr;
    bytes = used = 0;
    HIP_OK(hipHostMalloc(reinterpret_cast<void**>(&base), n, hipHostMallocDefault));
    bytes = n;
  }
};

}  // namespace

struct ppocr_hip_engine {
  ppocr_hip_ctx* ctx = nullptr;
  std::string detector_path, recognizer_path;
  ppocr_engine_options options{};
  size_t classes = 0, dictionary_len = 0;
  std::vector<Cached> detectors, recognizers;
  ppocr_hip_model* shared_weights = nullptr;  // any live recognizer plan
  PinnedStage stage;
  ~ppocr_hip_engine() {
    // Queued downloads may still target the staging area and queued graphs
    // may still run the cached plans.
    if (ctx) try {
        ppocr::sync_context(ctx);
      } catch (const std::exception&) {
      }
  }
};

struct ppocr_ocr_result {
  uint32_t source_size[2] = {0, 0};
  uint32_t detector_input_size[2] = {0, 0};
  std::vector<ppocr_ocr_line> lines;
  std::vector<int32_t> tokens;
};

namespace {

ppocr_hip_model* cached_model(ppocr_hip_engine* e, std::vector<Cached>& cache, size_t limit, const size_t shape[4],
                              bool detector) {
  for (Cached& c : cache)
    if (std::equal(shape, shape + 4, c.shape)) return c.model->m;
  if (cache.size() == limit) {
    ppocr::sync_context(e->ctx);  // queued batches may still run the evicted plan
    if (!detector && e->shared_weights == cache.front().model->m) e->shared_weights = nullptr;
    cache.erase(cache.begin());
    if (!detector && !e->shared_weights && !cache.empty()) e->shared_weights = cache.front().model->m;
  }
  ppocr_hip_model* m = nullptr;
  const ppocr_engine_options& o = e->options;
  if (detector) {
    check(ppocr_hip_detector_load(e->ctx, e->detector_path.c_str(), o.detector_size, shape, o.precision, &m));
  } else if (o.greedy) {
    check(ppocr_hip_recognizer_load_greedy(e->ctx, e->recognizer_path.c_str(), o.recognizer_size, shape,
                                           o.precision, e->shared_weights, &m));
  } else {
    check(ppocr_hip_recognizer_load(e->ctx, e->recognizer_path.c_str(), o.recognizer_size, shape, o.precision,
                                    e->shared_weights, &m));
  }
  Cached c;
  std::copy(shape, shape + 4, c.shape);
  c.model = std::make_unique<ModelHandle>(m);
  cache.push_back(std::move(c));
  if (!detector && !e->shared_weights) e->shared_weights = m;
  return m;
}

// Per-step (class, probability) of full probability rows: the argmax (ties
// -> last) and its value, as decode_ctc_greedy_for_input reads them.
std::vector<float> steps_from_rows(const std::vector<float>& rows, size_t items, size_t t, size_t v) {
  std::vector<float> steps(items * t * 2);
  for (size_t r = 0; r < items * t; ++r) {
    const float* row = rows.data() + r * v;
    size_t best = 0;
    for (size_t c = 1; c < v; ++c)
      if (!total_less(row[c], row[best])) best = c;
    steps[2 * r] = (float)best;
    steps[2 * r + 1] = row[best];
  }
  return steps;
}

}  // namespace

extern "C" {

void ppocr_engine_default_options(ppocr_engine_options* o) {
  if (!o) return;
  o->detector_size = PPOCR_SIZE_TINY;
  o->recognizer_size = PPOCR_SIZE_TINY;
  o->precision = PPOCR_F32;
  ppocr_db_default_options(&o->postprocess);
  o->detector_max_side = 736;
  o->greedy = 1;
}

ppocr_status ppocr_hip_engine_load(ppocr_hip_ctx* ctx, const char* detector_path, const char* recognizer_path,
                                   size_t dictionary_len, const ppocr_engine_options* options,
                                   ppocr_hip_engine** out) {
  return ppocr::guarded([&] {
    if (!ctx || !detector_path || !recognizer_path || !out) ppocr::raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    *out = nullptr;
    auto e = std::make_unique<ppocr_hip_engine>();
    ppocr_engine_default_options(&e->options);
    if (options) e->options = *options;
    const ppocr_engine_options& o = e->options;
    if (o.detector_size < PPOCR_SIZE_MEDIUM || o.detector_size > PPOCR_SIZE_TINY ||
        o.recognizer_size < PPOCR_SIZE_MEDIUM || o.recognizer_size > PPOCR_SIZE_TINY)
      ppocr::raise(PPOCR_ERR_INVALID_INPUT, "unknown model size");
    // OcrOptions::validate (src/ocr.rs:317-327).
    ppocr::db_options(&o.postprocess);
    if (o.precision != PPOCR_F32 && o.precision != PPOCR_BF16) ppocr::raise(PPOCR_ERR_INVALID_INPUT, "unknown precision");
    // validate_recognizer_dictionary (src/ocr.rs:691-700).
    e->classes = o.recognizer_size == PPOCR_SIZE_TINY ? 6906 : 18710;
    if (e->classes != dictionary_len + 1 && e->classes != dictionary_len + 2)
      ppocr::raise(PPOCR_ERR_INVALID_INPUT, "recognizer has " + std::to_string(e->classes) +
                                                " output classes, but the dictionary has " +
                                                std::to_string(dictionary_len) + " entries");
    e->dictionary_len = dictionary_len;
    e->ctx = ctx;
    e->detector_path = detector_path;
    e->recognizer_path = recognizer_path;
    *out = e.release();
  });
}

void ppocr_hip_engine_free(ppocr_hip_engine* engine) { delete engine; }

ppocr_status ppocr_hip_engine_recognize(ppocr_hip_engine* e, const uint8_t* rgb, uint32_t width, uint32_t height,
                                        ppocr_ocr_result** out) {
  return ppocr::guarded([&] {
    if (!e || !out) ppocr::raise(PPOCR_ERR_INVALID_INPUT, "null argument");
    *out = nullptr;
    auto result = std::make_unique<ppocr_ocr_result>();
    result->source_size[0] = width;
    result->source_size[1] = height;
    ImageHandle image;
    check(ppocr_hip_upload_rgb(e->ctx, width, height, rgb, (size_t)width * height * 3, &image.p));

    // Detection (DetectorInputPlan::new, run_detector, extract_detections).
    uint32_t iw = 0, ih = 0;
    const uint32_t max_side = e->options.detector_max_side;
    check(ppocr_detector_input_plan(width, height, max_side ? &max_side : nullptr, &iw, &ih));
    result->detector_input_size[0] = iw;
    result->detector_input_size[1] = ih;
    const size_t det_shape[4] = {1, 3, ih, iw};
    ppocr_hip_model* det = cached_model(e, e->detectors, DETECTOR_CACHE_LIMIT, det_shape, true);
    const float corners[8] = {0.0f, 0.0f, (float)width, 0.0f, (float)width, (float)height, 0.0f, (float)height};
    const ppocr_detector_transform tr{width, height, iw, ih};
    size_t count = 0, total = 0;
    const size_t cap = e->options.postprocess.max_boxes;
    std::vector<ppocr_detection> dets(cap);
    check(ppocr_hip_detect_image(det, image.p, corners, 1, &tr, &e->options.postprocess, dets.data(), cap, &count,
                                 &total));
    dets.resize(std::min(total, cap));

    // Recognition order: ascending aspect ratio, stable (src/ocr.rs:541-545).
    std::vector<size_t> order(dets.size());
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) {
      return total_less(aspect_ratio(dets[a].polygon), aspect_ratio(dets[b].polygon));
    });
    std::vector<std::vector<int32_t>> tokens(dets.size());
    std::vector<float> scores(dets.size(), 0.0f);
    auto decode = [&](const float* steps, size_t start, size_t n, size_t t, const std::vector<size_t>& content,
                      size_t input_width) {
      std::vector<int32_t> buf(t);
      for (size_t i = 0; i < n; ++i) {
        size_t emitted = 0;
        float score = 0.0f;
        check(ppocr_ctc_greedy_decode(&steps[2 * t * i], t, e->classes, e->dictionary_len, content[i], input_width,
                                      buf.data(), &emitted, &score));
        tokens[order[start + i]].assign(buf.begin(), buf.begin() + emitted);
        scores[order[start + i]] = score;
      }
    };
    // Greedy batches are queued back to back on the stream and decoded once
    // it has drained: one wait per page instead of two per batch.
    struct Queued {
      size_t start, n, t, input_width;
      std::vector<size_t> content;
      const float* steps;
    };
    std::vector<Queued> queued;
    auto drain = [&] {
      if (queued.empty()) return;
      ppocr::sync_context(e->ctx);
      for (const Queued& q : queued) {
        for (size_t i = 0; i < q.n * q.t * 2; ++i)
          if (!std::isfinite(q.steps[i])) ppocr::raise(PPOCR_ERR_GPU, "model output contains non-finite values");
        decode(q.steps, q.start, q.n, q.t, q.content, q.input_width);
      }
      queued.clear();
      e->stage.used = 0;
    };
    // Declared after `image`, so it runs first on every exit: no queued
    // batch outlives the page, its device image or its staging.
    struct DrainGuard {
      ppocr_hip_ctx* ctx;
      ~DrainGuard() {
        try {
          ppocr::sync_context(ctx);
        } catch (const std::exception&) {
        }
      }
    } guard{e->ctx};
    e->stage.used = 0;  // the previous page's guard drained the stream
    for (size_t start = 0; start < order.size(); start += RECOGNIZER_BATCH_SIZE) {
      const size_t n = std::min(RECOGNIZER_BATCH_SIZE, order.size() - start);
      std::vector<float> quads(8 * n);
      for (size_t i = 0; i < n; ++i) memcpy(&quads[8 * i], dets[order[start + i]].polygon, 8 * sizeof(float));
      size_t input_width = 0;
      check(ppocr_recognizer_batch_width(quads.data(), n, &input_width));
      std::vector<size_t> content(n);
      for (size_t i = 0; i < n; ++i) check(ppocr_recognition_input_plan(&quads[8 * i], input_width, &content[i]));
      const size_t rec_shape[4] = {n, 3, 48, input_width};
      ppocr_hip_model* rec = cached_model(e, e->recognizers, RECOGNIZER_CACHE_LIMIT, rec_shape, false);
      size_t oshape[4], rank = 0;
      check(ppocr_hip_output_shape(rec, oshape, &rank));
      const size_t t = oshape[1];
      if (e->options.greedy) {
        const size_t packet = ppocr::packet_bytes(n), out_bytes = n * t * 2 * sizeof(float);
        const size_t need = PinnedStage::round(packet) + PinnedStage::round(out_bytes);
        if (e->stage.used + need > e->stage.bytes) {
          drain();
          if (need > e->stage.bytes) e->stage.reserve(std::max(need, (size_t)1 << 20));
        }
        char* geo = e->stage.take(packet);
        float* steps = reinterpret_cast<float*>(e->stage.take(out_bytes));
        ppocr::enqueue_forward_image(rec, image.p, quads.data(), content.data(), n, geo, steps, n * t * 2);
        queued.push_back(Queued{start, n, t, input_width, content, steps});
      } else {
        std::vector<float> rows(n * t * e->classes);
        check(ppocr_hip_forward_image(rec, image.p, quads.data(), content.data(), n, rows.data(), rows.size()));
        const std::vector<float> steps = steps_from_rows(rows, n, t, e->classes);
        decode(steps.data(), start, n, t, content, input_width);
      }
    }
    drain();
    for (size_t i = 0; i < dets.size(); ++i) {
      ppocr_ocr_line line;
      memcpy(line.polygon, dets[i].polygon, sizeof line.polygon);
      line.detection_score = dets[i].score;
      line.recognition_score = scores[i];
      line.token_offset = result->tokens.size();
      line.token_count = tokens[i].size();
      result->tokens.insert(result->tokens.end(), tokens[i].begin(), tokens[i].end());
      result->lines.push_back(line);
    }
    *out = result.release();
  });
}

const ppocr_ocr_line* ppocr_ocr_result_lines(const ppocr_ocr_result* r, size_t* count) {
  if (count) *count = r ? r->lines.size() : 0;
  return r && !r->lines.empty() ? r->lines.data() : nullptr;
}

const int32_t* ppocr_ocr_result_tokens(const ppocr_ocr_result* r, size_t* count) {
  if (count) *count = r ? r->tokens.size() : 0;
  return r && !r->tokens.empty() ? r->tokens.data() : nullptr;
}

void ppocr_ocr_result_sizes(const ppocr_ocr_result* r, uint32_t source_size[2], uint32_t detector_input_size[2]) {
  if (!r) return;
  if (source_size) std::copy(r->source_size, r->source_size + 2, source_size);
  if (detector_input_size) std::copy(r->detector_input_size, r->detector_input_size + 2, detector_input_size);
}

void ppocr_ocr_result_free(ppocr_ocr_result* r) { delete r; }

}  // extern "C"
