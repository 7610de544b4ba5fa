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

// Thread-local message of the last failed C-ABI call (ppocr_hip_last_error).
std::string& last_error();

// Runs `f` as the body of a C-ABI entry point: no exception crosses the ABI;
// errors become their status code and the thread's last-error message.
template <typename F>
ppocr_status guarded(F&& f) {
  try {
    f();
    last_error().clear();
    return PPOCR_OK;
  } catch (const Error& e) {
    last_error() = e.what();
    return e.code;
  } catch (const std::bad_alloc&) {
    last_error() = "host allocation failed";
    return PPOCR_ERR_GPU;
  } catch (const std::exception& e) {
    last_error() = e.what();
    return PPOCR_ERR_GPU;
  }
}

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

inline size_t dtype_size(int dt) { return dt == DT_BF16 ? 2 : 4; }

// A view of an NHWC activation inside one planned buffer.  `off` is the
// element offset of channel 0 of pixel 0 (a channel slice of a wider tensor
// has off = first channel and ps = the wide tensor's channel count); `dt`
// is the storage type of the buffer's elements.
struct View {
  int buf = -1;
  size_t off = 0;
  int n = 0, h = 0, w = 0, c = 0, ps = 0;
  int dt = DT_F32;
  size_t pixels() const { return (size_t)n * h * w; }
};

struct Buffer {
  size_t bytes = 0;
  size_t arena_off = 0;  // bytes
  int first = -1, last = -1;
  std::string name;
  int dt = DT_F32;  // element storage type
};

struct Exec {
  char* arena = nullptr;
  const char* weights = nullptr;
  const std::vector<Buffer>* bufs = nullptr;
  void* ptr(const View& v) const { return arena + (*bufs)[v.buf].arena_off + v.off * dtype_size(v.dt); }
  float* fptr(const View& v) const { return static_cast<float*>(ptr(v)); }
  // Weight blob offsets are in bytes; SIZE_MAX means "absent".
  const void* wv(size_t off) const { return off == SIZE_MAX ? nullptr : weights + off; }
  const float* w(size_t off) const { return static_cast<const float*>(wv(off)); }
};

struct Op {
  std::string name;
  std::string kernel;
  double flops = 0.0, bytes = 0.0;
  int bound = 0;  // 0 HBM, 1 matrix cores, 2 fp32 vector ALU
  std::vector<int> reads, writes;
  std::function<void(const Exec&, hipStream_t)> launch;
  // bf16 plans: the values this op rounds to bf16 and the weights it takes
  // in bf16, by name.  With rounds_set false the rounded values are the bf16
  // buffers the op writes (plan_rounding_points); `exact` ops (maxima,
  // copies) round nothing.
  std::vector<std::string> rounds, bf16_weights;
  bool rounds_set = false, exact = false;
};

struct Plan {
  std::vector<Buffer> bufs;
  std::vector<Op> ops;
  std::vector<uint8_t> weights;  // packed host weights, byte blob (uploaded once)
  int staging = -1;              // fp32 NCHW input buffer (written by the host copy)
  View input;                    // NHWC4 model input
  int output = -1;               // fp32 output buffer
  size_t output_elems = 0;
  std::vector<size_t> output_shape;
  size_t arena_bytes = 0, unplanned_bytes = 0;
  bool detector = true;
  int dt = DT_F32;  // activation storage type
};

// Builds the plan of one model for a fixed input shape; `dt` selects fp32 or
// bf16 activation storage.  A `greedy` recognizer ends in the classifier
// fused with per-step greedy CTC decoding (output [N, T, 2]: class index,
// probability) instead of the softmax probabilities [N, T, V].  Both forms
// pack the same weight blob.
Plan build_detector(const SafeTensors& st, int size, const size_t nchw[4], int dt);
Plan build_recognizer(const SafeTensors& st, int size, const size_t nchw[4], int dt, bool greedy);

// Every point where a plan rounds to its bf16 storage type, in op order:
// "A <value>" for each activation value rounded (a bf16 buffer's name when
// one op writes it, else the writing op's name, or the op's explicit list)
// and "W <layer>" for each layer whose weights are bf16.  Empty for fp32
// plans.
std::vector<std::string> plan_rounding_points(const Plan& plan);

// Postprocess options (defaults when null) after
// DetectorPostprocessOptions::validate (src/ocr.rs:250-268).
ppocr_db_options db_options(const ppocr_db_options* o);

// Queued image forward for the engine's batch loop (no C-ABI counterpart):
// the checks and work of ppocr_hip_forward_image, with nothing waited for.
// `packet` (packet_bytes(n) bytes) and `out` must be pinned host memory
// (hipHostMalloc) left untouched until sync_context returns: the geometry
// upload reads `packet` and the output download writes `out` when the stream
// reaches them.
size_t packet_bytes(size_t n);
void enqueue_forward_image(ppocr_hip_model* model, const ppocr_hip_image* image, const float* corners,
                           const size_t* content_w, size_t n, char* packet, float* out, size_t out_cap);
// Waits for all work queued on the context's stream.
void sync_context(ppocr_hip_ctx* ctx);

// Lifetime-based offset packing of the plan's buffers into one arena
// (the reference's ArenaAllocator::compact_layout, src/gpu/runtime.rs:414-557).
void plan_arena(Plan& plan);

}  // namespace ppocr
