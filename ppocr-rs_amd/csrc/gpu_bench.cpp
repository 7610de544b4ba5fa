// ppocr-gpu-bench: benchmark one PP-OCRv6 model on the gfx950 backend.
//
// The command-line contract of the reference's `ppocr-gpu-bench`
// (src/bin/ppocr-gpu-bench.rs:45-88) and its shared benchmark module
// (src/bin/benchmark.rs): the same flags (`BenchmarkArgs`, :13-57, and the
// model-store flags of src/bin/model_store.rs:6-19), the same deterministic
// input (:126-134), little-endian f32 input/reference/dump files
// (:136-159), the same `key: value` report (:188-227) and reference
// comparison (:229-285).  It drives the backend only through the C ABI of
// include/ppocr_hip.h, as a Rust binding would.
//
// Differences, all additive: `--batch N` (the reference benchmarks batch 1
// only) and `--precision f32|bf16`.  Models resolve from `--model`, or from
// `<model-dir>/<size>-<kind>/model.safetensors` (src/models.rs:325-344)
// when that file is already cached: this program never downloads, so
// `--offline` changes nothing and `--verify-models`, which needs the pinned
// catalog's digests, is refused.
#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>
#include <sys/stat.h>
#include <vector>

#include "../../include/ppocr_hip.h"

namespace {

struct Fail : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// Usage error: clap prints it with the usage line and exits with status 2.
struct Usage : std::runtime_error {
  using std::runtime_error::runtime_error;
};

const char* kUsage =
    "Usage: ppocr-gpu-bench --kind <KIND> [OPTIONS]\n"
    "\n"
    "Benchmark one PP-OCRv6 model on the gfx950 (MI355X) backend\n"
    "\n"
    "Options:\n"
    "  --kind <KIND>          Model role to benchmark [possible values: det, rec]\n"
    "  --model-size <SIZE>    Released model tier [default: tiny] [possible values: medium, small, tiny]\n"
    "  --model <MODEL>        Explicit Safetensors file. Omit to use the model cache\n"
    "  --model-dir <DIR>      Directory where model packages are stored [env: PPOCR_MODEL_DIR] [default: models]\n"
    "  --offline              Fail when the model is not already cached (always the case here)\n"
    "  --verify-models        Recompute model hashes (needs the pinned catalog; refused here)\n"
    "  --height <HEIGHT>      Input height. Defaults to 416 for detector and 48 for recognizer\n"
    "  --width <WIDTH>        Input width. Defaults to 736 for detector and 320 for recognizer\n"
    "  --input <INPUT>        Little-endian F32 input file. Omit for deterministic generated input\n"
    "  --reference <FILE>     Compare the final output with a little-endian F32 reference file\n"
    "  --dump <FILE>          Write the final output as little-endian F32 values\n"
    "  --warmup <N>           Number of untimed warmup runs [default: 5]\n"
    "  --runs <N>             Number of timed runs [default: 30]\n"
    "  --batch <N>            Batch size (no reference counterpart) [default: 1]\n"
    "  --precision <P>        Storage precision (no reference counterpart) [default: f32] [possible values: f32, bf16]\n"
    "  --device <N>           HIP device ordinal [default: 0]\n"
    "  -h, --help             Print help\n";

struct Args {
  std::string kind;  // "det" | "rec"
  std::string model_size = "tiny";
  std::string model;
  std::string model_dir;
  bool offline = false, verify_models = false;
  long height = -1, width = -1;
  std::string input, reference, dump;
  long warmup = 5, runs = 30, batch = 1;
  std::string precision = "f32";
  int device = 0;
};

long parse_count(const std::string& flag, const std::string& v) {
  if (v.empty() || v[0] == '-' || v[0] == '+') throw Usage("invalid value '" + v + "' for '" + flag + "'");
  errno = 0;
  char* end = nullptr;
  const unsigned long long x = std::strtoull(v.c_str(), &end, 10);
  if (errno || *end || x > (unsigned long long)__LONG_MAX__)
    throw Usage("invalid value '" + v + "' for '" + flag + "'");
  return (long)x;
}

Args parse(int argc, char** argv) {
  Args a;
  if (const char* e = std::getenv("PPOCR_MODEL_DIR")) a.model_dir = e;
  if (a.model_dir.empty()) a.model_dir = "models";
  for (int i = 1; i < argc; ++i) {
    std::string flag = argv[i], value;
    bool has_value = false;
    const size_t eq = flag.find('=');
    if (flag.rfind("--", 0) == 0 && eq != std::string::npos) {
      value = flag.substr(eq + 1);
      flag = flag.substr(0, eq);
      has_value = true;
    }
    if (flag == "-h" || flag == "--help") {
      std::fputs(kUsage, stdout);
      std::exit(0);
    }
    if (flag == "--offline" || flag == "--verify-models") {
      if (has_value) throw Usage("unexpected value '" + value + "' for '" + flag + "'");
      (flag == "--offline" ? a.offline : a.verify_models) = true;
      continue;
    }
    if (!has_value) {
      if (i + 1 >= argc) throw Usage("a value is required for '" + flag + "' but none was supplied");
      value = argv[++i];
    }
    if (flag == "--kind") {
      if (value != "det" && value != "rec") throw Usage("invalid value '" + value + "' for '--kind <KIND>'");
      a.kind = value;
    } else if (flag == "--model-size") {
      if (value != "tiny" && value != "small" && value != "medium")
        throw Usage("invalid value '" + value + "' for '--model-size <MODEL_SIZE>'");
      a.model_size = value;
    } else if (flag == "--model") {
      a.model = value;
    } else if (flag == "--model-dir") {
      a.model_dir = value;
    } else if (flag == "--height") {
      a.height = parse_count(flag, value);
    } else if (flag == "--width") {
      a.width = parse_count(flag, value);
    } else if (flag == "--input") {
      a.input = value;
    } else if (flag == "--reference") {
      a.reference = value;
    } else if (flag == "--dump") {
      a.dump = value;
    } else if (flag == "--warmup") {
      a.warmup = parse_count(flag, value);
    } else if (flag == "--runs") {
      a.runs = parse_count(flag, value);
    } else if (flag == "--batch") {
      a.batch = parse_count(flag, value);
    } else if (flag == "--precision") {
      if (value != "f32" && value != "bf16") throw Usage("invalid value '" + value + "' for '--precision'");
      a.precision = value;
    } else if (flag == "--device") {
      a.device = (int)parse_count(flag, value);
    } else {
      throw Usage("unexpected argument '" + std::string(argv[i]) + "' found");
    }
  }
  if (a.kind.empty()) throw Usage("the following required arguments were not provided:\n  --kind <KIND>");
  if (a.offline && a.verify_models)
    throw Usage("the argument '--offline' cannot be used with '--verify-models'");
  return a;
}

// BenchmarkArgs::input_shape (src/bin/benchmark.rs:60-70).
std::vector<size_t> input_shape(const Args& a) {
  if (a.runs <= 0) throw Fail("--runs must be positive");
  const bool det = a.kind == "det";
  const long h = a.height >= 0 ? a.height : (det ? 416 : 48);
  const long w = a.width >= 0 ? a.width : (det ? 736 : 320);
  if (h <= 0) throw Fail("--height must be positive");
  if (w <= 0) throw Fail("--width must be positive");
  if (a.batch <= 0) throw Fail("--batch must be positive");
  return {(size_t)a.batch, 3, (size_t)h, (size_t)w};
}

// deterministic_input (src/bin/benchmark.rs:126-134): a 32-bit LCG, the top
// 24 bits of each state scaled to [-1, 1] in f32 arithmetic.
std::vector<float> deterministic_input(size_t length) {
  std::vector<float> v(length);
  uint32_t state = 0x243f6a88u;
  for (size_t i = 0; i < length; ++i) {
    state = state * 1664525u + 1013904223u;
    const float unit = (float)(state >> 8) / (float)0x00ffffff;
    v[i] = unit * 2.0f - 1.0f;
  }
  return v;
}

// read_f32 (src/bin/benchmark.rs:136-148): exactly `expected` values.
std::vector<float> read_f32(const std::string& path, size_t expected) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw Fail("read " + path + ": " + std::strerror(errno));
  std::vector<char> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  if (bytes.size() != expected * sizeof(float))
    throw Fail(path + " must contain " + std::to_string(expected) + " F32 values, found " +
               std::to_string(bytes.size()) + " bytes");
  std::vector<float> v(expected);
  for (size_t i = 0; i < expected; ++i) {
    const unsigned char* b = reinterpret_cast<const unsigned char*>(bytes.data()) + 4 * i;
    const uint32_t u = (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24;
    std::memcpy(&v[i], &u, 4);
  }
  return v;
}

// write_f32 (src/bin/benchmark.rs:150-158).
void write_f32(const std::string& path, const std::vector<float>& values) {
  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  if (!f) throw Fail("create " + path + ": " + std::strerror(errno));
  for (float x : values) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    const unsigned char b[4] = {(unsigned char)u, (unsigned char)(u >> 8), (unsigned char)(u >> 16),
                                (unsigned char)(u >> 24)};
    f.write(reinterpret_cast<const char*>(b), 4);
  }
  f.flush();
  if (!f) throw Fail("write " + path);
}

// validate_output (src/bin/benchmark.rs:160-167).
void validate_output(const std::vector<float>& v) {
  if (v.empty()) throw Fail("model output is empty");
  for (float x : v)
    if (!std::isfinite(x)) throw Fail("model output contains non-finite values");
}

// Rust's `{:.9e}`: mantissa with nine decimals, exponent without sign or
// padding ("5.000000000e-1", "1.234500000e3").  glibc's %.9e rounds the
// exact binary value as Rust does; only the exponent is rewritten.
std::string sci9(double x) {
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.9e", x);
  std::string s = buf;
  const size_t e = s.find('e');
  if (e == std::string::npos) return s;
  const int exp = std::atoi(s.c_str() + e + 1);
  return s.substr(0, e + 1) + std::to_string(exp);
}

std::string fixed(double x, int digits) {
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.*f", digits, x);
  return buf;
}

std::string dims(const std::vector<size_t>& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

// percentile (src/bin/benchmark.rs:322-325): nearest rank, index rounded
// half away from zero.
double percentile(const std::vector<double>& sorted, double p) {
  const size_t i = (size_t)std::round((double)(sorted.size() - 1) * p);
  return sorted[i];
}

// Last index of the maximum (Rust's max_by keeps the last of equal
// elements, src/bin/benchmark.rs:287-293).
size_t argmax(const float* v, size_t n) {
  size_t best = 0;
  for (size_t i = 1; i < n; ++i)
    if (!(v[i] < v[best])) best = i;
  return best;
}

void check(ppocr_status s) {
  if (s != PPOCR_OK) {
    const char* m = ppocr_hip_last_error();
    throw Fail(m && *m ? m : ("backend error " + std::to_string((int)s)));
  }
}

bool is_file(const std::string& p) {
  struct stat st;
  return ::stat(p.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

// resolve_model_path (src/bin/benchmark.rs:113-124) without the downloader.
std::string resolve_model_path(const Args& a) {
  if (!a.model.empty()) return a.model;
  const std::string name = a.model_size + "-" + a.kind;
  if (a.verify_models)
    throw Fail("--verify-models needs the pinned model catalog, which this program does not carry; pass --model");
  const std::string path = a.model_dir + "/" + name + "/model.safetensors";
  if (!is_file(path))
    throw Fail(name + " is missing in " + a.model_dir + "/" + name +
               "; this program does not download models: pass --model or fill the cache");
  return path;
}

struct Handles {
  ppocr_hip_ctx* ctx = nullptr;
  ppocr_hip_model* model = nullptr;
  ~Handles() {
    if (model) ppocr_hip_model_free(model);
    if (ctx) ppocr_hip_destroy(ctx);
  }
};

int run(const Args& a) {
  const std::vector<size_t> shape = input_shape(a);
  const size_t length = shape[0] * shape[1] * shape[2] * shape[3];
  const std::vector<float> input = a.input.empty() ? deterministic_input(length) : read_f32(a.input, length);
  const std::string model_path = resolve_model_path(a);
  const ppocr_model_size size =
      a.model_size == "tiny" ? PPOCR_SIZE_TINY : a.model_size == "small" ? PPOCR_SIZE_SMALL : PPOCR_SIZE_MEDIUM;
  const ppocr_precision precision = a.precision == "bf16" ? PPOCR_BF16 : PPOCR_F32;

  Handles h;
  check(ppocr_hip_create(a.device, &h.ctx));
  if (a.kind == "det")
    check(ppocr_hip_detector_load(h.ctx, model_path.c_str(), size, shape.data(), precision, &h.model));
  else
    check(ppocr_hip_recognizer_load(h.ctx, model_path.c_str(), size, shape.data(), precision, nullptr, &h.model));
  size_t oshape[4] = {0, 0, 0, 0}, rank = 0;
  check(ppocr_hip_output_shape(h.model, oshape, &rank));
  std::vector<size_t> out_shape(oshape, oshape + rank);
  size_t out_len = 1;
  for (size_t d : out_shape) out_len *= d;

  std::vector<float> output(out_len);
  check(ppocr_hip_forward(h.model, input.data(), input.size(), output.data(), output.size()));
  validate_output(output);
  float lo = INFINITY, hi = -INFINITY;
  double sum = 0.0;
  for (float x : output) {
    lo = std::fmin(lo, x);
    hi = std::fmax(hi, x);
    sum += (double)x;
  }
  std::vector<double> samples((size_t)a.runs);
  check(ppocr_hip_benchmark(h.model, input.data(), input.size(), (size_t)a.warmup, (size_t)a.runs, samples.data()));

  double total = 0.0;
  for (double s : samples) total += s;
  const double average_ms = total / (double)samples.size();
  std::vector<double> sorted = samples;
  std::sort(sorted.begin(), sorted.end());

  std::printf("backend: gpu\n");
  std::printf("kind: %s\n", a.kind.c_str());
  std::printf("model: %s\n", model_path.c_str());
  std::printf("input_shape: %s\n", dims(shape).c_str());
  std::printf("output_shape: %s\n", dims(out_shape).c_str());
  std::printf("output_min: %s\n", sci9(lo).c_str());
  std::printf("output_max: %s\n", sci9(hi).c_str());
  std::printf("output_sum: %s\n", sci9(sum).c_str());
  std::printf("warmup: %ld\n", a.warmup);
  std::printf("runs: %ld\n", a.runs);
  std::printf("average_ms: %s\n", fixed(average_ms, 3).c_str());
  std::printf("p50_ms: %s\n", fixed(percentile(sorted, 0.50), 3).c_str());
  std::printf("p90_ms: %s\n", fixed(percentile(sorted, 0.90), 3).c_str());
  std::printf("p95_ms: %s\n", fixed(percentile(sorted, 0.95), 3).c_str());
  std::printf("throughput: %s\n", fixed(1000.0 / average_ms, 2).c_str());
  if (a.batch > 1) std::printf("items_per_second: %s\n", fixed(1000.0 * (double)a.batch / average_ms, 2).c_str());

  if (!a.reference.empty()) {
    // report_reference (src/bin/benchmark.rs:229-285).
    const std::vector<float> expected = read_f32(a.reference, output.size());
    for (float x : expected)
      if (!std::isfinite(x)) throw Fail("reference contains non-finite values");
    float max_abs = 0.0f;
    double total_abs = 0.0;
    for (size_t i = 0; i < output.size(); ++i) {
      const float d = std::fabs(output[i] - expected[i]);
      max_abs = std::fmax(max_abs, d);
      total_abs += (double)d;
    }
    std::printf("reference_max_abs: %s\n", sci9(max_abs).c_str());
    std::printf("reference_mean_abs: %s\n", sci9(total_abs / (double)output.size()).c_str());
    if (a.kind == "det") {
      size_t mismatches = 0;
      for (size_t i = 0; i < output.size(); ++i) mismatches += (output[i] >= 0.5f) != (expected[i] >= 0.5f);
      std::printf("reference_threshold_0.5_mismatches: %zu\n", mismatches);
    } else {
      const size_t classes = out_shape.back();
      if (classes == 0) throw Fail("recognizer class axis is empty");
      size_t mismatches = 0;
      for (size_t r = 0; r + classes <= output.size(); r += classes)
        mismatches += argmax(&output[r], classes) != argmax(&expected[r], classes);
      std::printf("reference_argmax_mismatches: %zu\n", mismatches);
    }
  }
  if (!a.dump.empty()) {
    write_f32(a.dump, output);
    std::printf("dump: %s\n", a.dump.c_str());
  }
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const Args a = parse(argc, argv);
    return run(a);
  } catch (const Usage& e) {
    std::fprintf(stderr, "error: %s\n\n%s", e.what(), kUsage);
    return 2;
  } catch (const std::exception& e) {
    std::fflush(stdout);
    std::fprintf(stderr, "Error: %s\n", e.what());
    return 1;
  }
}
