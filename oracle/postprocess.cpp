// CPU restatement of the reference's DB detector postprocess (test
// infrastructure only: the parity checker for the device postprocess).
//
// Follows src/ocr.rs step by step, in the reference's types and order:
//   extract_detections        src/ocr.rs:723-790
//   collect_component (BFS)   src/ocr.rs:1006-1054
//   fit_rotated_box           src/ocr.rs:1056-1118
//   sort_detections           src/ocr.rs:1120-1131
//   polygon_center            src/ocr.rs:1133-1138
//   DetectorTransform::map_*  src/ocr.rs:66-74
// The f32 sums run in the BFS visiting order, as the reference's do.
#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <deque>
#include <vector>

namespace {

struct Pt {
  float x, y;
};

struct Det {
  Pt poly[4];
  float score;
  float anisotropy;  // diagnostic: |(2 cov_xy, cov_xx - cov_yy)| / (cov_xx + cov_yy)
};

struct Component {
  std::vector<Pt> points;
  double score_sum = 0.0;
};

Component collect_component(const float* values, size_t width, size_t cw, size_t ch, size_t sx, size_t sy,
                            float threshold, std::vector<uint8_t>& visited) {
  static const int NB[8][2] = {{-1, -1}, {0, -1}, {1, -1}, {-1, 0}, {1, 0}, {-1, 1}, {0, 1}, {1, 1}};
  Component c;
  std::deque<std::pair<size_t, size_t>> queue;
  queue.push_back({sx, sy});
  visited[sy * cw + sx] = 1;
  while (!queue.empty()) {
    auto [x, y] = queue.front();
    queue.pop_front();
    c.points.push_back({(float)x + 0.5f, (float)y + 0.5f});
    c.score_sum += (double)values[y * width + x];
    for (const auto& d : NB) {
      const long nx = (long)x + d[0], ny = (long)y + d[1];
      if (nx < 0 || ny < 0 || nx >= (long)cw || ny >= (long)ch) continue;
      const size_t ni = (size_t)ny * cw + (size_t)nx;
      if (!visited[ni] && values[(size_t)ny * width + (size_t)nx] >= threshold) {
        visited[ni] = 1;
        queue.push_back({(size_t)nx, (size_t)ny});
      }
    }
  }
  return c;
}

float dot(Pt a, Pt b) {
  const float p = a.x * b.x;
  const float q = a.y * b.y;
  return p + q;
}
Pt add(Pt a, Pt b) { return {a.x + b.x, a.y + b.y}; }
Pt scale(Pt a, float f) { return {a.x * f, a.y * f}; }

void fit_rotated_box(const std::vector<Pt>& pts, float unclip, Pt out[4], float* anisotropy) {
  const float count = (float)pts.size();
  float sx = 0.0f, sy = 0.0f;
  for (const Pt& p : pts) sx += p.x;
  for (const Pt& p : pts) sy += p.y;
  Pt center{sx / count, sy / count};
  float cxx = 0.0f, cxy = 0.0f, cyy = 0.0f;
  for (const Pt& p : pts) {
    const float dx = p.x - center.x, dy = p.y - center.y;
    cxx = cxx + dx * dx;
    cxy = cxy + dx * dy;
    cyy = cyy + dy * dy;
  }
  const float angle = 0.5f * std::atan2(2.0f * cxy, cxx - cyy);
  Pt axis{std::cos(angle), std::sin(angle)};
  if (axis.x < 0.0f || (std::fabs(axis.x) < 1.1920929e-7f && axis.y < 0.0f)) axis = {-axis.x, -axis.y};
  const Pt normal{-axis.y, axis.x};
  float min_a = INFINITY, max_a = -INFINITY, min_n = INFINITY, max_n = -INFINITY;
  for (const Pt& p : pts) {
    const Pt d{p.x - center.x, p.y - center.y};
    const float a = dot(d, axis), n = dot(d, normal);
    min_a = std::fmin(min_a, a);
    max_a = std::fmax(max_a, a);
    min_n = std::fmin(min_n, n);
    max_n = std::fmax(max_n, n);
  }
  const float axis_center = (min_a + max_a) * 0.5f;
  const float normal_center = (min_n + max_n) * 0.5f;
  const float half_axis = ((max_a - min_a + 1.0f) * unclip) * 0.5f;
  const float half_normal = ((max_n - min_n + 1.0f) * unclip) * 0.5f;
  const Pt c = add(center, add(scale(axis, axis_center), scale(normal, normal_center)));
  out[0] = add(c, add(scale(axis, -half_axis), scale(normal, -half_normal)));
  out[1] = add(c, add(scale(axis, half_axis), scale(normal, -half_normal)));
  out[2] = add(c, add(scale(axis, half_axis), scale(normal, half_normal)));
  out[3] = add(c, add(scale(axis, -half_axis), scale(normal, half_normal)));
  const double tr = (double)cxx + (double)cyy;
  *anisotropy = tr > 0.0 ? (float)(std::hypot(2.0 * cxy, (double)cxx - cyy) / tr) : 0.0f;
}

Pt polygon_center(const Pt* p) {
  float sx = 0.0f, sy = 0.0f;
  for (int i = 0; i < 4; ++i) sx += p[i].x;
  for (int i = 0; i < 4; ++i) sy += p[i].y;
  return {sx / 4.0f, sy / 4.0f};
}

// f32::total_cmp on finite values: -1, 0, 1 (-0.0 orders before +0.0).
int total_cmp(float a, float b) {
  if (a < b) return -1;
  if (a > b) return 1;
  return (int)std::signbit(b) - (int)std::signbit(a);
}

// sort_detections: stable sort by center y, center x, then score.
void sort_detections(std::vector<Det>& d) {
  std::stable_sort(d.begin(), d.end(), [](const Det& l, const Det& r) {
    const Pt a = polygon_center(l.poly), b = polygon_center(r.poly);
    if (int c = total_cmp(a.y, b.y)) return c < 0;
    if (int c = total_cmp(a.x, b.x)) return c < 0;
    return total_cmp(l.score, r.score) < 0;
  });
}

}  // namespace

extern "C" {

// values: [height][width] probabilities of one image; transform: source w,
// source h, content w, content h.  Writes `count` records of 10 floats
// (polygon x0 y0 .. x3 y3, score, anisotropy) into out (capacity cap).
// Returns 0, or -1 on invalid arguments.
int oracle_extract_detections(const float* values, int height, int width, const uint32_t transform[4],
                              float binary_threshold, float box_threshold, size_t min_area, float unclip_ratio,
                              size_t max_boxes, float* out, size_t cap, size_t* count) {
  if (!values || !transform || !count || height <= 0 || width <= 0) return -1;
  if (!(binary_threshold >= 0.0f && binary_threshold <= 1.0f) || !(box_threshold >= 0.0f && box_threshold <= 1.0f) ||
      min_area == 0 || max_boxes == 0 || !std::isfinite(unclip_ratio) || unclip_ratio <= 0.0f)
    return -1;
  for (uint32_t i = 0; i < 4; ++i)
    if (transform[i] == 0) return -1;
  const size_t H = (size_t)height, W = (size_t)width;
  for (size_t i = 0; i < H * W; ++i)
    if (!std::isfinite(values[i])) return -1;
  const float src_w = (float)transform[0], src_h = (float)transform[1];
  const float con_w = (float)transform[2], con_h = (float)transform[3];
  const size_t cw = std::min<size_t>(transform[2], W), ch = std::min<size_t>(transform[3], H);
  std::vector<uint8_t> visited(cw * ch, 0);
  std::vector<Det> dets;
  for (size_t y = 0; y < ch; ++y) {
    for (size_t x = 0; x < cw; ++x) {
      if (visited[y * cw + x] || values[y * W + x] < binary_threshold) continue;
      Component c = collect_component(values, W, cw, ch, x, y, binary_threshold, visited);
      if (c.points.size() < min_area) continue;
      const float score = (float)(c.score_sum / (double)c.points.size());
      if (score < box_threshold) continue;
      Det d;
      fit_rotated_box(c.points, unclip_ratio, d.poly, &d.anisotropy);
      for (Pt& p : d.poly) {
        p.x = std::clamp(p.x * src_w / con_w, 0.0f, src_w);
        p.y = std::clamp(p.y * src_h / con_h, 0.0f, src_h);
      }
      d.score = score;
      dets.push_back(d);
    }
  }
  sort_detections(dets);
  if (dets.size() > max_boxes) {
    std::stable_sort(dets.begin(), dets.end(), [](const Det& l, const Det& r) {
      if (int c = total_cmp(r.score, l.score)) return c < 0;
      const Pt a = polygon_center(l.poly), b = polygon_center(r.poly);
      if (int c = total_cmp(a.y, b.y)) return c < 0;
      return total_cmp(a.x, b.x) < 0;
    });
    dets.resize(max_boxes);
    sort_detections(dets);
  }
  *count = dets.size();
  for (size_t i = 0; i < dets.size() && i < cap && out; ++i) {
    float* o = out + 10 * i;
    for (int k = 0; k < 4; ++k) {
      o[2 * k] = dets[i].poly[k].x;
      o[2 * k + 1] = dets[i].poly[k].y;
    }
    o[8] = dets[i].score;
    o[9] = dets[i].anisotropy;
  }
  return 0;
}

}  // extern "C"
