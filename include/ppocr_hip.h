/*
 * ppocr_hip.h — C ABI of the MI355X (gfx950) backend for the PP-OCRv6
 * detector and recognizer.
 *
 * This is the drop-in boundary for the reference's `ppocr_rs::gpu` direct
 * model API (src/gpu/mod.rs:3-13).  Every entry point names the reference
 * item it replaces.  Plain pointers and sizes only; no exception or abort
 * crosses it; the library owns all device memory.  A handle may be used from
 * any thread but not concurrently: forward calls serialise on a per-context
 * mutex, as the reference's `Mutex<SharedWorkspace>` does
 * (src/gpu/runtime.rs:75, :1753-1758).
 */
#ifndef PPOCR_HIP_H
#define PPOCR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes, one per variant of the reference `gpu::Error`
 * (src/gpu/error.rs:9-45). */
typedef enum ppocr_status {
  PPOCR_OK = 0,
  PPOCR_ERR_READ_FILE = 1,
  PPOCR_ERR_SAFETENSORS = 2,
  PPOCR_ERR_TENSOR_NOT_FOUND = 3,
  PPOCR_ERR_UNSUPPORTED_DTYPE = 4,
  PPOCR_ERR_SHAPE_MISMATCH = 5,
  PPOCR_ERR_TENSOR_SIZE_OVERFLOW = 6,
  PPOCR_ERR_TENSOR_BYTE_LENGTH = 7,
  PPOCR_ERR_INVALID_TENSOR_RANGE = 8,
  PPOCR_ERR_INVALID_MODEL = 9,
  PPOCR_ERR_INVALID_INPUT = 10,
  PPOCR_ERR_GPU = 11
} ppocr_status;

/* `ModelSize` (src/models.rs), in the reference's declaration order. */
typedef enum ppocr_model_size {
  PPOCR_SIZE_MEDIUM = 0,
  PPOCR_SIZE_SMALL = 1,
  PPOCR_SIZE_TINY = 2
} ppocr_model_size;

/* Activation/weight storage precision.  F32 is the reference's arithmetic;
 * BF16 keeps bf16 weights and activations with fp32 accumulation. */
typedef enum ppocr_precision { PPOCR_F32 = 0, PPOCR_BF16 = 1 } ppocr_precision;

typedef struct ppocr_hip_ctx ppocr_hip_ctx;     /* `gpu::Gpu` */
typedef struct ppocr_hip_model ppocr_hip_model; /* `gpu::Detector` / `gpu::Recognizer` */
typedef struct ppocr_hip_image ppocr_hip_image; /* `gpu::GpuImage` */

/* Message of the last failed call on this thread (empty when none). */
const char* ppocr_hip_last_error(void);

/* Replaces `Gpu::new` (src/gpu/runtime.rs:94-167): opens `device`, creates
 * the stream and the shared activation arena. */
ppocr_status ppocr_hip_create(int device, ppocr_hip_ctx** out);
void ppocr_hip_destroy(ppocr_hip_ctx* ctx);

/* `GpuInfo` (src/gpu/runtime.rs:17-21): the adapter's name, backend and
 * device type, plus what a HIP device adds (architecture, compute units,
 * memory).  Strings are NUL-terminated and cut to fit. */
typedef struct ppocr_gpu_info {
  char name[256];    /* marketing name, e.g. "AMD Instinct MI355X" */
  char backend[16];  /* "HIP" (the reference reports its wgpu backend) */
  char arch[64];     /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int device;        /* HIP device index of the context */
  int integrated;    /* 1 for an integrated GPU (wgpu DeviceType::IntegratedGpu), 0 for a discrete one */
  int compute_units;
  int wavefront_size;
  size_t total_memory; /* bytes of device memory */
} ppocr_gpu_info;

/* Replaces `Gpu::info` (src/gpu/runtime.rs:169-171). */
ppocr_status ppocr_hip_device_info(const ppocr_hip_ctx* ctx, ppocr_gpu_info* out);

/* Replaces `Detector::load` (src/gpu/model.rs:50-93): loads a safetensors
 * file, checks the tier's tensor count (350/271/271), folds BatchNorm, packs
 * the weights, and plans the graph for the fixed input shape `nchw`
 * ([N, 3, H, W], N > 0, H and W >= 32 and divisible by 32,
 * src/gpu/model.rs:268-276). */
ppocr_status ppocr_hip_detector_load(ppocr_hip_ctx* ctx, const char* safetensors_path, ppocr_model_size size,
                                     const size_t nchw[4], ppocr_precision precision, ppocr_hip_model** out);

/* Replaces `Recognizer::load` / `load_with_shared_weights`
 * (src/gpu/model.rs:156-220): [N, 3, 48, W] with W >= 32 and divisible by 4
 * (src/gpu/model.rs:278-286).  When `share_weights` is a recognizer loaded
 * from the same file, its device weights are reused. */
ppocr_status ppocr_hip_recognizer_load(ppocr_hip_ctx* ctx, const char* safetensors_path, ppocr_model_size size,
                                       const size_t nchw[4], ppocr_precision precision,
                                       const ppocr_hip_model* share_weights, ppocr_hip_model** out);

/* A recognizer whose classifier is fused with the per-step half of greedy
 * CTC decoding (`decode_ctc_greedy_for_input`, src/ocr.rs:800-853, which
 * takes each time step's argmax class, ties to the last index, and that
 * class's softmax probability).  Loaded like ppocr_hip_recognizer_load; its
 * output is [N, T, 2] floats, (class index, probability) per time step, in
 * place of the [N, T, V] probabilities, so the probability tensor is never
 * written to HBM or copied to the host.  `share_weights` may be either form
 * of recognizer loaded from the same file.  No counterpart in the reference,
 * whose recognizer always returns the full probabilities (src/gpu/model.rs:222-237). */
ppocr_status ppocr_hip_recognizer_load_greedy(ppocr_hip_ctx* ctx, const char* safetensors_path,
                                              ppocr_model_size size, const size_t nchw[4], ppocr_precision precision,
                                              const ppocr_hip_model* share_weights, ppocr_hip_model** out);

void ppocr_hip_model_free(ppocr_hip_model* model);

/* Output shape of `ModelOutput` (src/gpu/model.rs:37-41): detector
 * [N, 1, H, W] (rank 4), recognizer [N, T, V] (rank 3). */
ppocr_status ppocr_hip_output_shape(const ppocr_hip_model* model, size_t shape[4], size_t* rank);

/* Replaces `Detector::forward` / `Recognizer::forward`
 * (src/gpu/model.rs:95-114, :222-237): host NCHW float input of exactly the
 * planned shape; writes the compact output (detector sigmoid probabilities,
 * recognizer softmax probabilities) into `out` (capacity `out_cap` floats).
 * Non-finite input or output is an error, as src/gpu/runtime.rs:1979-1983,
 * :2217-2219. */
ppocr_status ppocr_hip_forward(ppocr_hip_model* model, const float* nchw, size_t len, float* out, size_t out_cap);

/* Replaces `Gpu::upload_rgb` (src/gpu/runtime.rs:174-229): RGB8, row-major
 * HWC, `width * height * 3` bytes. */
ppocr_status ppocr_hip_upload_rgb(ppocr_hip_ctx* ctx, uint32_t width, uint32_t height, const uint8_t* rgb,
                                  size_t len, ppocr_hip_image** out);
void ppocr_hip_image_free(ppocr_hip_image* image);

/* Replaces `Detector::forward_image` / `Recognizer::forward_image` with
 * `ImagePreprocess` (src/gpu/model.rs:116-138, :239-256,
 * src/gpu/runtime.rs:52-70, :2086-2155).  The preprocessing follows the
 * reference CPU path (src/preprocess.rs:78-123), including the integer
 * rounding of the bilinear sample.  `corners` holds N quads of four (x, y)
 * source points (top-left, top-right, bottom-right, bottom-left);
 * `content_widths` holds N widths (NULL: the full canvas).  Unlike the
 * reference, whose device path accepts N = 1 only (src/gpu/runtime.rs:2016),
 * every crop of a recognizer batch is rectified on the device. */
ppocr_status ppocr_hip_forward_image(ppocr_hip_model* model, const ppocr_hip_image* image, const float* corners,
                                     const size_t* content_widths, size_t n, float* out, size_t out_cap);

/* Device preprocessing alone (`prepare_detector` / `prepare_recognizer`,
 * src/preprocess.rs:37-76): writes [3, canvas_h, canvas_w] NCHW floats,
 * BGR-normalised with the detector (`detector` != 0) or recognizer
 * statistics, columns >= content_width zero. */
ppocr_status ppocr_hip_preprocess(ppocr_hip_ctx* ctx, const ppocr_hip_image* image, const float corners[8],
                                  size_t canvas_w, size_t canvas_h, size_t content_width, int detector,
                                  float* out_nchw);

/* Replaces `Detector::benchmark` / `Recognizer::benchmark`
 * (src/gpu/model.rs:140-148, src/gpu/runtime.rs:1798-1830): uploads once,
 * runs `warmup` untimed passes, then `runs` timed passes, each timed from
 * launch to completion; writes one duration in milliseconds per run. */
ppocr_status ppocr_hip_benchmark(ppocr_hip_model* model, const float* nchw, size_t len, size_t warmup, size_t runs,
                                 double* samples_ms);

/* Throughput form of the benchmark: inputs already resident in HBM,
 * `runs` passes launched back to back and synchronised once; writes the
 * total elapsed milliseconds.  No counterpart in the reference, which
 * synchronises every pass. */
ppocr_status ppocr_hip_benchmark_stream(ppocr_hip_model* model, const float* nchw, size_t len, size_t warmup,
                                        size_t runs, double* total_ms);

/* Per-kernel timing record; replaces the PPOCR_GPU_PROFILE timestamp report
 * (src/gpu/runtime.rs:1832-1933).  `flops` and `bytes` are the algorithmic
 * work of one launch (2 x MACs; inputs + weights + outputs read or written
 * once, logical channels). */
typedef struct ppocr_kernel_stat {
  char name[64];
  char kernel[32];
  double avg_ms;
  double flops;
  double bytes;
  int bound; /* 0: HBM-bound, 1: matrix-core bound, 2: fp32 vector-ALU bound */
} ppocr_kernel_stat;

/* Runs `runs` passes with a HIP event around every launch (on the stream the
 * kernels run on) and reports the mean duration per launch.  `count`
 * receives the number of launches in one pass; at most `cap` are written. */
ppocr_status ppocr_hip_profile(ppocr_hip_model* model, const float* nchw, size_t len, size_t runs,
                               ppocr_kernel_stat* stats, size_t cap, size_t* count);

/* Memory report (PPOCR_GPU_MEMORY_REPORT, src/gpu/runtime.rs:1486-1492,
 * :1737-1742): arena bytes of this model's plan, the sum of its buffers
 * without reuse, and device weight bytes. */
ppocr_status ppocr_hip_memory_report(const ppocr_hip_model* model, size_t* arena_bytes, size_t* unplanned_bytes,
                                     size_t* weight_bytes);

/* ---- DB detector postprocess on the device. */

/* `DetectorPostprocessOptions` (src/ocr.rs:231-269); defaults 0.2, 0.4, 3,
 * 1.4, 1000 (ppocr_db_default_options).  Thresholds must lie in [0, 1],
 * min_area and max_boxes be at least 1, unclip_ratio be finite and > 0. */
typedef struct ppocr_db_options {
  float binary_threshold;
  float box_threshold;
  size_t min_area;
  float unclip_ratio;
  size_t max_boxes;
} ppocr_db_options;

/* `DetectorTransform` (src/ocr.rs:32-74): the source image size and the
 * content size it was resized to inside the detector canvas.  All non-zero. */
typedef struct ppocr_detector_transform {
  uint32_t source_width, source_height, content_width, content_height;
} ppocr_detector_transform;

/* `Detection` (src/ocr.rs:225-229): four (x, y) corners in source pixels,
 * and the mean probability of the component. */
typedef struct ppocr_detection {
  float polygon[8];
  float score;
} ppocr_detection;

void ppocr_db_default_options(ppocr_db_options* options);

/* `extract_detections` (src/ocr.rs:723-790) over `n` host probability maps
 * [n][height][width], computed on the device: pixels >= binary_threshold
 * inside each content rectangle, 8-connected components with at least
 * min_area pixels and mean probability >= box_threshold, the rotated box of
 * each (principal axis, extents, unclip), mapped to source coordinates,
 * sorted by centre y, x, score (`sort_detections`, :1120-1131) and cut to
 * max_boxes by score.  `counts[i]` receives image i's detection count and
 * `total` their sum; up to `cap` detections are written to `out`, image by
 * image.  `options` NULL means the defaults. */
ppocr_status ppocr_hip_db_postprocess(ppocr_hip_ctx* ctx, const float* prob, size_t n, size_t height, size_t width,
                                      const ppocr_detector_transform* transforms, const ppocr_db_options* options,
                                      ppocr_detection* out, size_t cap, size_t* counts, size_t* total);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): ppocr_hip_db_postprocess with the same arguments and
 * results, whose staged maps and work arrays live in a static device scratch
 * of 64 MiB per GPU, held until the process ends; it calls no hipMalloc or
 * hipFree.  Maps needing more scratch (about 51 bytes per pixel, e.g. four
 * 416 x 736 maps) are rejected with PPOCR_ERR_INVALID_INPUT.  All calls on
 * one GPU share its scratch, so calls on one GPU serialise (also across
 * contexts): a call holds the device's scratch from staging the maps until
 * its detections are read back. */
ppocr_status ppocr_hip_db_postprocess_static(ppocr_hip_ctx* ctx, const float* prob, size_t n, size_t height,
                                             size_t width, const ppocr_detector_transform* transforms,
                                             const ppocr_db_options* options, ppocr_detection* out, size_t cap,
                                             size_t* counts, size_t* total);

/* Detector forward followed by the device postprocess on its output, which
 * never leaves the device: `GpuOcrRuntime::run_detector` +
 * `extract_detections` (src/ocr.rs:608-646, :723-790).  One transform per
 * image of the planned batch; outputs as ppocr_hip_db_postprocess. */
ppocr_status ppocr_hip_detect(ppocr_hip_model* detector, const float* nchw, size_t len,
                              const ppocr_detector_transform* transforms, const ppocr_db_options* options,
                              ppocr_detection* out, size_t cap, size_t* counts, size_t* total);

/* As ppocr_hip_detect, with the input rectified from a device image (one
 * quad per image of the batch, as ppocr_hip_forward_image). */
ppocr_status ppocr_hip_detect_image(ppocr_hip_model* detector, const ppocr_hip_image* image, const float* corners,
                                    size_t n, const ppocr_detector_transform* transforms,
                                    const ppocr_db_options* options, ppocr_detection* out, size_t cap,
                                    size_t* counts, size_t* total);

/* ---- End-to-end OCR engine (the `OcrBackend` arm, src/ocr.rs:276-281). */

typedef struct ppocr_hip_engine ppocr_hip_engine; /* `OcrEngine` with its GPU runtime */
typedef struct ppocr_ocr_result ppocr_ocr_result; /* `OcrResult` (src/ocr.rs:343-351) */

/* `OcrOptions` (src/ocr.rs:285-299) for this backend.  detector_max_side 0
 * means `None` (the model's own resize policy); greedy != 0 runs the
 * recognizer with the fused greedy-CTC classifier (only per-step class and
 * probability leave the device), 0 with the full probabilities. */
typedef struct ppocr_engine_options {
  ppocr_model_size detector_size;
  ppocr_model_size recognizer_size;
  ppocr_precision precision;
  ppocr_db_options postprocess;
  uint32_t detector_max_side;
  int greedy;
} ppocr_engine_options;

/* `OcrLine` (src/ocr.rs:331-341): polygon in source pixels, detector score,
 * the recognised text as `token_count` class indices starting at
 * `token_offset` of the result's token array (class c is dictionary entry
 * c - 1, or a space for the implicit last class), recognition score. */
typedef struct ppocr_ocr_line {
  float polygon[8];
  float detection_score;
  float recognition_score;
  size_t token_offset;
  size_t token_count;
} ppocr_ocr_line;

/* Defaults of `OcrOptions::default` (src/ocr.rs:300-314): tiny / tiny,
 * default postprocess, max side 736; plus F32 and greedy decoding. */
void ppocr_engine_default_options(ppocr_engine_options* options);

/* `OcrEngine::load` (src/ocr.rs:416-494) with the GPU runtime: validates the
 * options and that the recognizer's class count is dictionary_len + 1 or + 2
 * (`validate_recognizer_dictionary`, :691-700).  Models are loaded lazily per
 * input shape and cached: 2 detector and 4 recognizer plans, oldest evicted
 * first, all recognizer plans sharing one copy of the weights
 * (`GpuOcrRuntime`, :608-689).  `options` NULL means the defaults. */
ppocr_status ppocr_hip_engine_load(ppocr_hip_ctx* ctx, const char* detector_path, const char* recognizer_path,
                                   size_t dictionary_len, const ppocr_engine_options* options,
                                   ppocr_hip_engine** out);
void ppocr_hip_engine_free(ppocr_hip_engine* engine);

/* `OcrEngine::recognize` / `recognize_with` (src/ocr.rs:497-600) on an RGB8
 * image (row-major HWC, width * height * 3 bytes).  The result is read with
 * the accessors below and released with ppocr_ocr_result_free. */
ppocr_status ppocr_hip_engine_recognize(ppocr_hip_engine* engine, const uint8_t* rgb, uint32_t width,
                                        uint32_t height, ppocr_ocr_result** out);
const ppocr_ocr_line* ppocr_ocr_result_lines(const ppocr_ocr_result* result, size_t* count);
const int32_t* ppocr_ocr_result_tokens(const ppocr_ocr_result* result, size_t* count);
void ppocr_ocr_result_sizes(const ppocr_ocr_result* result, uint32_t source_size[2],
                            uint32_t detector_input_size[2]);
void ppocr_ocr_result_free(ppocr_ocr_result* result);

/* ---- Host-side geometry and decoding around the device path (no GPU).
 * Errors are PPOCR_ERR_INVALID_INPUT with the message in
 * ppocr_hip_last_error(). */

/* Detector input size for a `width` x `height` image: `DetectorInputPlan::new`
 * (src/ocr.rs:86-101) with `default_detector_ratio` (:173-184) when
 * `max_side` is NULL and min(max_side / max(w, h), 1) otherwise, each side
 * then rounded by `aligned_dimension` (:186-195) to the nearest multiple of
 * 32 (at least 32).  1920 x 1080 with max_side 736 gives 736 x 416. */
ppocr_status ppocr_detector_input_plan(uint32_t width, uint32_t height, const uint32_t* max_side,
                                       uint32_t* input_width, uint32_t* input_height);

/* Canvas width of a recognizer batch: `recognizer_batch_width`
 * (src/ocr.rs:206-219) over `n` quads (corners [n][4][2]): the largest
 * content width, at least 320, rounded up to a multiple of 4. */
ppocr_status ppocr_recognizer_batch_width(const float* corners, size_t n, size_t* width);

/* Content width of one crop on a canvas of `input_width`:
 * `recognition_input_plan` (src/ocr.rs:154-171) with
 * `bounded_crop_dimensions` (:1145-1156) and `scaled_recognizer_width`
 * (:197-204), i.e. ceil(48 w / h) of the bounded crop size. */
ppocr_status ppocr_recognition_input_plan(const float corners[8], size_t input_width, size_t* content_width);

/* The sequential half of `decode_ctc_greedy_for_input` (src/ocr.rs:800-853)
 * on one item's `steps` ([T][2], as written by a greedy recognizer):
 * collapses repeats and blanks over the first ceil(content_width T /
 * input_width) steps and writes the emitted class indices (1..classes-1;
 * with an implicit space class, classes - 1 is the space) to `tokens`
 * (capacity T), their count, and the score exp(mean ln p) (0 when nothing is
 * emitted).  `classes` must be dictionary_len + 1 or + 2. */
ppocr_status ppocr_ctc_greedy_decode(const float* steps, size_t time_steps, size_t classes, size_t dictionary_len,
                                     size_t content_width, size_t input_width, int32_t* tokens, size_t* n_tokens,
                                     float* score);

#ifdef __cplusplus
}
#endif

#endif /* PPOCR_HIP_H */
