// Host-side OCR geometry and greedy CTC collapse (include/ppocr_hip.h).
//
// These are the integer/f32 input-plan rules and the sequential tail of
// greedy CTC decoding that sit either side of the device path: the plan
// decides the tensor shapes the models are loaded for, and the collapse turns
// the device's per-step (class, probability) pairs into tokens and a score.
// Arithmetic follows the reference's types step by step (f64 ratios, f32
// edge lengths, u32 integer division); products are not contracted.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <string>

#include "runtime.h"

using ppocr::guarded;

namespace {

[[noreturn]] void fail(const std::string& msg) { ppocr::raise(PPOCR_ERR_INVALID_INPUT, msg); }

constexpr double DETECTOR_LIMIT_SIDE = 736.0;   // src/ocr.rs:24
constexpr double DETECTOR_MAX_SIDE = 4000.0;    // src/ocr.rs:26
constexpr uint32_t RECOGNIZER_INPUT_HEIGHT = 48;  // src/ocr.rs:17
constexpr size_t RECOGNIZER_INPUT_WIDTH = 320;    // src/ocr.rs:18
constexpr float MAX_RECTIFIED_EDGE = 4096.0f;     // src/ocr.rs:20
constexpr float MAX_RECTIFIED_PIXELS = 8000000.0f;  // src/ocr.rs:21
constexpr float PROBABILITY_EPSILON = 1e-8f;        // src/ocr.rs:23

// default_detector_ratio (src/ocr.rs:173-184).
double default_detector_ratio(uint32_t width, uint32_t height) {
  const double min_side = (double)std::min(width, height);
  double ratio = min_side < DETECTOR_LIMIT_SIDE ? DETECTOR_LIMIT_SIDE / min_side : 1.0;
  const double max_side = (double)std::max(width, height);
  if (max_side * ratio > DETECTOR_MAX_SIDE) ratio = DETECTOR_MAX_SIDE / max_side;
  return ratio;
}

// aligned_dimension (src/ocr.rs:186-195): nearest multiple of 32, at least 32.
uint32_t aligned_dimension(double value) {
  if (!std::isfinite(value) || value <= 0.0) fail("invalid resized image dimension " + std::to_string(value));
  const double units = std::max(std::round(value / 32.0), 1.0);
  if (units > (double)(std::numeric_limits<uint32_t>::max() / 32))
    fail("resized image dimension " + std::to_string(value) + " is too large");
  return (uint32_t)units * 32;
}

// distance (src/ocr.rs:1215-1217), f32 with separate roundings.
float distance(const float* a, const float* b) {
  const float dx = a[0] - b[0], dy = a[1] - b[1];
  const float sq = dx * dx;
  const float sq2 = dy * dy;
  return std::sqrt(sq + sq2);
}

// bounded_crop_dimensions (src/ocr.rs:1145-1156).
void bounded_crop_dimensions(float width, float height, uint32_t* w, uint32_t* h) {
  if (!std::isfinite(width) || !std::isfinite(height) || width <= 0.0f || height <= 0.0f)
    fail("text polygon has an invalid crop size " + std::to_string(width) + " by " + std::to_string(height));
  const float edge_scale = std::min(MAX_RECTIFIED_EDGE / std::max(width, height), 1.0f);
  const float area = width * height;
  const float pixel_scale = std::min(std::sqrt(MAX_RECTIFIED_PIXELS / area), 1.0f);
  const float scale = std::min(edge_scale, pixel_scale);
  const float sw = width * scale, sh = height * scale;
  *w = (uint32_t)std::clamp(std::round(sw), 1.0f, MAX_RECTIFIED_EDGE);
  *h = (uint32_t)std::clamp(std::round(sh), 1.0f, MAX_RECTIFIED_EDGE);
}

// scaled_recognizer_width (src/ocr.rs:197-204): ceil(48 w / h), at least 1.
size_t scaled_recognizer_width(uint32_t width, uint32_t height) {
  const uint64_t num = (uint64_t)RECOGNIZER_INPUT_HEIGHT * width;
  if (num > std::numeric_limits<uint32_t>::max()) fail("recognizer content width overflow");
  return (size_t)std::max<uint64_t>((num + height - 1) / height, 1);
}

// Crop width and height of a quad: the longer of each pair of opposite edges
// (src/ocr.rs:158-160, :209-211), bounded.
void crop_dimensions(const float* q, uint32_t* w, uint32_t* h) {
  const float width = std::max(distance(q + 0, q + 2), distance(q + 6, q + 4));
  const float height = std::max(distance(q + 0, q + 6), distance(q + 2, q + 4));
  bounded_crop_dimensions(width, height, w, h);
}

void check_finite(const float* v, size_t n, const char* what) {
  if (!v) fail(std::string(what) + " pointer is null");
  for (size_t i = 0; i < n; ++i)
    if (!std::isfinite(v[i])) fail(std::string(what) + " contain non-finite values");
}

}  // namespace

extern "C" {

ppocr_status ppocr_detector_input_plan(uint32_t width, uint32_t height, const uint32_t* max_side,
                                       uint32_t* input_width, uint32_t* input_height) {
  return guarded([&] {
    if (!input_width || !input_height) fail("null output pointer");
    if (width == 0 || height == 0) fail("detector transform dimensions must be non-zero");
    double ratio;
    if (max_side) {
      if (*max_side == 0) fail("detector maximum side must be positive");
      ratio = std::min((double)*max_side / (double)std::max(width, height), 1.0);
    } else {
      ratio = default_detector_ratio(width, height);
    }
    const uint32_t w = aligned_dimension((double)width * ratio);
    const uint32_t h = aligned_dimension((double)height * ratio);
    *input_width = w;
    *input_height = h;
  });
}

ppocr_status ppocr_recognizer_batch_width(const float* corners, size_t n, size_t* width) {
  return guarded([&] {
    if (!width) fail("null output pointer");
    if (n) check_finite(corners, n * 8, "corners");
    size_t maximum = RECOGNIZER_INPUT_WIDTH;
    for (size_t i = 0; i < n; ++i) {
      uint32_t w, h;
      crop_dimensions(corners + 8 * i, &w, &h);
      maximum = std::max(maximum, scaled_recognizer_width(w, h));
    }
    *width = (maximum + 3) / 4 * 4;
  });
}

ppocr_status ppocr_recognition_input_plan(const float corners[8], size_t input_width, size_t* content_width) {
  return guarded([&] {
    if (!content_width) fail("null output pointer");
    check_finite(corners, 8, "corners");
    uint32_t w, h;
    crop_dimensions(corners, &w, &h);
    const size_t content = scaled_recognizer_width(w, h);
    if (content > input_width) fail("recognizer crop exceeds its batch canvas");
    *content_width = content;
  });
}

ppocr_status ppocr_ctc_greedy_decode(const float* steps, size_t time_steps, size_t classes, size_t dictionary_len,
                                     size_t content_width, size_t input_width, int32_t* tokens, size_t* n_tokens,
                                     float* score) {
  return guarded([&] {
    if (!tokens || !n_tokens || !score) fail("null output pointer");
    if (time_steps == 0 || classes == 0) fail("recognizer output must have time steps and classes");
    const bool implicit_space = classes == dictionary_len + 2;
    if (classes != dictionary_len + 1 && !implicit_space)
      fail("recognizer output has " + std::to_string(classes) + " classes, but the dictionary has " +
           std::to_string(dictionary_len) + " entries; expected dictionary entries plus the CTC blank class");
    if (content_width == 0 || content_width > input_width)
      fail("recognizer content width " + std::to_string(content_width) + " is outside 1..=" +
           std::to_string(input_width));
    check_finite(steps, time_steps * 2, "recognizer steps");
    size_t valid = (content_width * time_steps + input_width - 1) / input_width;
    valid = std::clamp<size_t>(valid, 1, time_steps);
    double log_score = 0.0;
    size_t emitted = 0, previous = 0;
    for (size_t t = 0; t < valid; ++t) {
      const float c = steps[2 * t];
      if (c < 0.0f || c >= (float)classes || c != std::floor(c)) fail("recognizer step class out of range");
      const size_t cls = (size_t)c;
      if (cls != 0 && cls != previous) {
        tokens[emitted++] = (int32_t)cls;
        const float p = std::clamp(steps[2 * t + 1], 0.0f, 1.0f);
        log_score += std::log((double)std::max(p, PROBABILITY_EPSILON));
      }
      previous = cls;
    }
    *n_tokens = emitted;
    *score = emitted == 0 ? 0.0f : (float)std::exp(log_score / (double)emitted);
  });
}

}  // extern "C"
