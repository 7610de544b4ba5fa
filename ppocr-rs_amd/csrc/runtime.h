// Host runtime of the MI355X backend: weights, plans, arena, sessions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/ppocr_hip.h"
#include "kernels.h"

namespace ppocr {

// Error carrying one of the C-ABI status codes (1:1 with the reference
// gpu::Error variants, src/gpu/error.rs:9-45).
struct Error : std::runtime_error {
  ppocr_status code;
  Error(ppocr_status c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] inline void raise(ppocr_status code, const std::string& msg) { throw Error(code, msg); }

#define HIP_OK(expr)                                                                                 \
  do {                                                                                               \
    hipError_t e_ = (expr);                                                                          \
    if (e_ != hipSuccess) ::ppocr::raise(PPOCR_ERR_GPU, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

// ------------------------------------------------------------------ weights

struct HostTensor {
  std::vector<int> shape;
  std::vector<float> v;
  size_t count() const {
    size_t n = 1;
    for (int d : shape) n *= (size_t)d;
    return n;
  }
};

// Safetensors file, F32 tensors only (src/gpu/weights.rs:28-86, :111-116).
class SafeTensors {
 public:
  static SafeTensors load(const std::string& path);
  size_t size() const { return tensors_.size(); }
  // VarBuilder::get with shape validation (src/gpu/weights.rs:247-319).
  HostTensor get(const std::string& name, const std::vector<int>& shape) const;
  bool contains(const std::string& name) const { return tensors_.count(name) != 0; }

 private:
  std::map<std::string, HostTensor> tensors_;
};

// ------------------------------------------------------------------ plans

// A view of an NHWC activation inside one planned buffer.  `off` is the
// element offset of channel 0 of pixel 0 (a channel slice of a wider tensor
// has off = first channel and ps = the wide tensor's channel count).
struct View {
  int buf = -1;
  size_t off = 0;
  int n = 0, h = 0, w = 0, c = 0, ps = 0;
  size_t pixels() const { return (size_t)n * h * w; }
};

struct Buffer {
  size_t elems = 0;
  size_t arena_off = 0;  // elements
  int first = -1, last = -1;
  std::string name;
};

struct Exec {
  float* arena = nullptr;
  const float* weights = nullptr;
  const std::vector<Buffer>* bufs = nullptr;
  float* ptr(const View& v) const { return arena + (*bufs)[v.buf].arena_off + v.off; }
  float* buf(int id) const { return arena + (*bufs)[id].arena_off; }
  const float* w(size_t off) const { return off == SIZE_MAX ? nullptr : weights + off; }
};

struct Op {
  std::string name;
  std::string kernel;
  double flops = 0.0, bytes = 0.0;
  int bound = 0;  // 0 HBM, 1 matrix cores
  std::vector<int> reads, writes;
  std::function<void(const Exec&, hipStream_t)> launch;
};

struct Plan {
  std::vector<Buffer> bufs;
  std::vector<Op> ops;
  std::vector<float> weights;  // packed host weights (uploaded once)
  int staging = -1;            // NCHW input buffer (written by the host copy)
  View input;                  // NHWC4 model input
  int output = -1;             // output buffer
  size_t output_elems = 0;
  std::vector<size_t> output_shape;
  size_t arena_elems = 0, unplanned_elems = 0;
  bool detector = true;
};

// Builds the plan of one model for a fixed input shape.
Plan build_detector(const SafeTensors& st, int size, const size_t nchw[4]);
Plan build_recognizer(const SafeTensors& st, int size, const size_t nchw[4]);

// Lifetime-based offset packing of the plan's buffers into one arena
// (the reference's ArenaAllocator::compact_layout, src/gpu/runtime.rs:414-557).
void plan_arena(Plan& plan);

}  // namespace ppocr
