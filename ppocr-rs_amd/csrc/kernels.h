// Kernel parameter blocks and host launchers of the gfx950 kernels.
//
// Activations live in one HBM arena in NHWC order: a tensor view is
// (pointer to channel 0 of pixel 0, N, H, W, C, pixel stride).  A pixel
// stride larger than C lets a producer write one channel slice of a wider
// tensor (the channel concats of the stem and the FPN are never copied).
// Activations are stored as fp32 or bf16 (`dt`); arithmetic is always fp32
// (bf16 MFMA products accumulate in fp32).  Small parameter tensors (biases,
// depthwise taps, SE and LayerNorm weights) stay fp32 in both precisions.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <mutex>
#include <string>

namespace ppocr {

enum DType : int { DT_F32 = 0, DT_BF16 = 1 };

// Activation codes: the epilogue set of the reference
// (src/gpu/runtime.rs:302-311, src/cpu/kernels/mod.rs:2376-2390).
enum Act : int {
  ACT_NONE = 0,
  ACT_RELU = 1,
  ACT_GELU = 2,
  ACT_SILU = 3,
  ACT_HSIG6 = 4,  // clamp(x/6 + 0.5, 0, 1): LCNet SE gate
  ACT_HSIG5 = 5,  // clamp(x/5 + 0.5, 0, 1): neck SE gate
  ACT_HSWISH = 6,
  ACT_SIGMOID = 7,
};

// Implicit-GEMM convolution on the matrix cores.
//   out[m, n] = act(sum_k A[m, k] * Wt[n, k] + bias[n])  (+ epilogue terms)
// m: output pixel (n_img, oy, ox); n: output channel; k = (ky*kw + kx)*C + c.
struct ConvParams {
  const void* in;
  int N, H, W, C, in_ps;
  void* out;
  int out_f32;  // store the output as fp32 whatever the activation type
  int Ho, Wo, Co, out_ps;
  const void* wt;  // packed [Co][ldw] in the activation type
  int ldw;         // = K (a multiple of 4)
  const float* bias;  // [Co] or null
  int kh, kw, sh, sw, pt, pl;
  int act;
  const float* in_gate;   // [N][C]: A[m, k] = x * g[n_img, c] (SE prologue)
  const void* res;        // residual added after the activation
  int res_ps;
  const float* res_gate;  // [N][Co]: residual term is res * g
  const void* up;         // nearest-upsample-add source [N, Ho/up_s, Wo/up_s, Co]
  int up_s, up_ps;
  int rep;           // write each output pixel as a rep x rep block (upsample on write)
  int rep_split;     // set by the launcher: workgroup z writes output row z of each rep x rep block only
  int out_h, out_w;  // dims of the tensor `out` points into (Ho*rep, Wo*rep)
  int dt;            // activation type of in / res / up / out
  // Greedy-CTC epilogue (classifier only; `out` unused, no other epilogue
  // terms): per row m and column tile j of conv_tile_cols() columns, the
  // tile's max logit, sum of exp(logit - max) and the last column holding the
  // max, stored as three planes [3][n_tiles][M] of floats.
  float* ctc_part;
  // Split K (splits > 1, from conv_split_k): workgroup row y of the grid
  // multiplies K slices [y*nk/splits, (y+1)*nk/splits) of its tile and
  // stores the raw fp32 sums to split_ws [splits][M][Co]; a second kernel
  // adds the splits in order and runs the epilogue.  Not combined with the
  // greedy-CTC epilogue.
  float* split_ws;
  int splits;
  // DB head tail (db_ch > 0): the GEMM is conv_up of the detector head as a
  // 1x1 conv whose column tap * db_ch + o is hidden channel o of 2x2 tap
  // `tap`; the epilogue adds the bias, applies ReLU, then conv_final (2x2
  // stride 2 to one channel: weights db_wf [db_ch][4], bias db_bf) and the
  // sigmoid, and writes the fp32 map `out` [N][4 Ho][4 Wo].  The tile width
  // must be a multiple of db_ch; no other epilogue terms.
  int db_ch;
  const float* db_wf;
  float db_bf;
  // Channel sums of the stored output for a squeeze-excitation that reads
  // it next ([P][Co] fp32, P = conv_se_blocks(): one row per tile row block
  // of a wave), or null.
  float* se_part;
};

// Depthwise k x k convolution (groups == C), 4 channels per lane.
struct DwParams {
  const void* in;
  int N, H, W, C, in_ps;
  void* out;
  int Ho, Wo, out_ps;
  const float* wt;  // [kh*kw][C]
  const float* bias;
  int kh, kw, sh, sw, pt, pl;
  int act;
  const void* res;  // out = res + act(dw(x) + b)
  int res_ps;
  int dt;
  // Per-block channel sums of the stored output for a squeeze-excitation
  // ([N][P][C] fp32, P = depthwise_se_blocks()), or null.
  float* se_part;
  // bf16 matrix-core operand fragments of the taps (depthwise_mfma_table),
  // or null; used when depthwise_uses_mfma() holds for the layer.
  const void* wtab;
  // Gate-residual prologue (gr_gate set; 5x5, 7x7 and 9x9 stride-1
  // layers): the conv's input is x = in + in * gr_gate[n] (two roundings,
  // as gate_residual_kernel) plus, with gr_up, the nearest 2x upsample of
  // gr_up [N][H/2][W/2] (pixel stride gr_up_ps), rounded to the storage
  // type; it is formed per tile from `in` and, with gr_out, also stored at
  // the layer's output pixels (pixel stride gr_out_ps).
  const float* gr_gate;
  const void* gr_up;
  int gr_up_ps;
  void* gr_out;
  int gr_out_ps;
};

// Squeeze-excitation gate: g[n, c] = gate_act(W2 relu(W1 mean(x) + b1) + b2).
struct SeParams {
  const void* in;
  int N, HW, C, in_ps;
  float* partial;  // [N][P][C] partial sums
  int P;           // pixel chunks per image
  const float* w1;  // [Cr][C] reduce weight
  const float* b1;
  const float* w2;  // [C][Cr] expand weight
  const float* b2;
  int Cr;
  int gate_act;
  float* hidden;  // [N][Cr]
  float* gate;    // [N][C]
  int dt;
};

void launch_conv(const ConvParams& p, hipStream_t s);
// Up to kConvMultiMax independent layers in one launch (first[i]: index of
// layer i's first tile, set by launch_conv_multi).  conv_multi_supported
// tells whether a set of layers can share one: the same kernel instance,
// no split K, upsample-on-write or DB-head / greedy-CTC epilogue, and no SE
// input gate.
constexpr int kConvMultiMax = 4;
struct ConvMulti {
  ConvParams p[kConvMultiMax];
  int first[kConvMultiMax];
  int count;
};
bool conv_multi_supported(const ConvParams* p, int count);
void launch_conv_multi(const ConvMulti& m, hipStream_t s);
// Layers whose depthwise launch can take the gate-residual prologue
// (DwParams::gr_gate): 5x5 / 7x7 / 9x9, stride 1 (with gr_up the map sides must
// be twice gr_up's).
bool depthwise_gate_residual_supported(int kh, int kw, int sh, int sw);

// Fused pointwise pair of an LCNet block (pair_gemm.hip), fp32, rows are
// pixels: x' = x * gate[image] (gate null: x' = x), h = GELU(x' W1^T + b1)
// kept on chip, out = h W2^T + b2 (+ x' when residual; Co == C).  C, H2
// and Co multiples of 16; weights packed [rows][ldw] as the conv GEMM's.
struct PairParams {
  const float* in;
  int in_ps;
  const float* gate;  // [N][C] or null
  int HW;             // pixels per image (the gate's image of a row)
  int M, C, H2, Co;
  const float* w1;
  int ldw1;
  const float* b1;
  const float* w2;
  int ldw2;
  const float* b2;
  int residual;
  float* out;
  int out_ps;
  // Depthwise prologue (dw_in set, no gate): the pair's input x is the 3x3
  // depthwise conv of dw_in [N][dw_h][dw_w] (pixel stride dw_ps), weights
  // [9][C], bias [C], stride (dw_sh, dw_sw), pads (dw_pt, dw_pl), no
  // activation, computed per tile and never stored; the pair's pixel grid
  // is HW pixels per image, dw_wo of them per row.
  const float* dw_in;
  int dw_ps, dw_h, dw_w, dw_wo, dw_sh, dw_sw, dw_pt, dw_pl;
  const float* dw_wt;
  const float* dw_b;
  // SE gate formed in the prologue (gate null, se_part set; one image,
  // pair_se_fold_supported): the channel means of x from its partial sums
  // se_part [se_P][C] over HW pixels, then act(W2 relu(W1 mean + b1) + b2)
  // with W1 [se_Cr][C] and W2 [C][se_Cr] packed densely.
  const float* se_part;
  int se_P, se_Cr, se_act;
  const float* se_w1;
  const float* se_b1;
  const float* se_w2;
  const float* se_b2;
};
bool pointwise_pair_supported(int C, int H2, int Co, int dt);
// Whether the pair kernel can form the SE gate of its input itself from P
// partial channel sums (N images, C channels, H2 hidden, Cr reduced ones).
bool pair_se_fold_supported(int N, int C, int H2, int Cr, int P);

// bf16 pointwise pair of an LCNet block (pair_bf16.hip): out = conv2(GELU(
// conv1(x * gate))) (+ x * gate), conv1 C -> 2C, conv2 2C -> C, one launch.
// x, out bf16 [M][ps]; gate fp32 [N][C] over HW pixels per image, or null;
// weights bf16 packed [rows][ldw], biases fp32.
struct PairBf16Params {
  const void* in;
  int in_ps;
  const float* gate;
  int HW;
  int M, C;
  const void* w1;  // [2C][ldw1]
  int ldw1;
  const float* b1;
  const void* w2;  // [C][ldw2]
  int ldw2;
  const float* b2;
  int residual;
  void* out;
  int out_ps;
};
bool pair_bf16_supported(int C, int H2, int Co);
// Compute units of the current device (256 when it cannot be queried),
// looked up once per device.
int device_cus();
std::string pair_bf16_kernel_name(const PairBf16Params& p);
void launch_pair_bf16(const PairBf16Params& p, hipStream_t s);

// LayerNorm fused into the linear layer that reads it (pair_gemm.hip), fp32:
// out[m][n] = act(sum_k LN(x[m])[k] w[n][k] + b[n]), LN with eps over K
// features (K a multiple of 4); weights packed [N][ldw].
struct LnLinearParams {
  const float* in;
  int in_ps;
  int M, K, N;
  const float* ln_w;
  const float* ln_b;
  float eps;
  const float* w;
  int ldw;
  const float* b;
  int act;
  float* out;
  int out_ps;
};
size_t ln_linear_lds(int K);
bool ln_linear_supported(int K, int N, int dt);
void launch_ln_linear(const LnLinearParams& p, hipStream_t s);
size_t pointwise_pair_lds(int C, int H2);
void launch_pointwise_pair(const PairParams& p, hipStream_t s);
// Name of the kernel instance launch_conv runs for p (tile, and the variant:
// 1x1 or k x k, gated, register-staged); the pointers of p are only tested
// for null and 16-byte alignment.
std::string conv_kernel_name(const ConvParams& p);
// Column width of that instance's tiles.
int conv_tile_cols(int M, int cols, int dt);
// Rows of the SE channel-sum array the conv leaves in se_part (single-image
// fp32 1x1 layers finished from registers), or 0 where it cannot.
int conv_se_blocks(const ConvParams& p);
// K splits for a convolution of M rows, Co columns and reduction depth K:
// more than 1 when its tiles alone would leave most of the 256 CUs idle and
// K is deep enough to divide (the workspace is splits * M * Co floats).
int conv_split_k(int M, int Co, int K, int dt);
// Merges the greedy-CTC partials of launch_conv into one (class, probability)
// pair per row: out[m] = {argmax (ties -> last index), softmax value of it}.
void launch_ctc_merge(const float* part, int M, int n_tiles, float* out, hipStream_t s);
void launch_depthwise(const DwParams& p, hipStream_t s);
// Blocks per image of the depthwise launch when it can leave the channel
// sums of its output for a squeeze-excitation (p.se_part), else 0.
int depthwise_se_blocks(const DwParams& p);
// Name of the kernel instance launch_depthwise picks; `groups8`: every
// pixel access (input, output, residual) starts on a whole group of 8
// channels.
const char* depthwise_kernel_name(int kh, int kw, int sh, int sw, int Ho, int dt = DT_F32, bool table = false,
                                  int C = 0, bool groups8 = true);
// bf16 layers with square stride-1 5x5, 7x7 or 9x9 kernels, at least 16
// output rows and a multiple of 8 channels run on the matrix cores when their
// taps come packed by depthwise_mfma_table (pack for Ho = 16: the rows are
// known at launch) and their pixel strides and addresses are in whole
// 8-channel (16-byte) groups.
bool depthwise_uses_mfma(int kh, int kw, int sh, int sw, int dt, int Ho, int C);
// Elements (bf16) of the packed taps of a c-channel k x k layer.
size_t depthwise_mfma_table_size(int c, int k);
// Packs taps w [c][k * k] (fp32) as [c][ky][lane 0..63][8] bf16: lane l holds
// w[ky][8 * (l / 16) + i - l % 16] for i = 0..7 (zero outside 0..k-1), the B
// fragment of a 16x16x32 product whose A rows are input rows and whose K
// runs over 32 input columns.
void depthwise_mfma_table(const float* w, int c, int k, uint16_t* out);
void launch_se(const SeParams& p, hipStream_t s);
// Stages 2 and 3 of launch_se from partial sums already in p.partial
// ([N][P][C], e.g. from the producing depthwise).
void launch_se_from_partials(const SeParams& p, hipStream_t s);
// Up to four gates from given partial sums in one launch (grid y = gate),
// for the FPN's per-level gates: each gate must take the one-workgroup path
// (se_multi_kind) and all of them the same kind.
constexpr int kSeMultiMax = 4;
struct SeMulti {
  SeParams p[kSeMultiMax];
  int count;
};
// 1 (small weights), 2 (one workgroup, larger weights) or 0 (not batchable).
int se_multi_kind(const SeParams& p);
void launch_se_multi(const SeMulti& m, hipStream_t s);
// Whether launch_se runs the gate as one kernel (small maps and weights; the
// partial and hidden arrays are then unused).
bool se_fused(const SeParams& p);

// NCHW fp32 (3 planes) -> NHWC with 4 channels (fourth channel zero).
void launch_nchw_to_nhwc4(const float* in, void* out, int N, int H, int W, int dt, hipStream_t s);

// Max pool 2x2, stride 1, pads (0,0,1,1) into a channel slice.
void launch_maxpool_same(const void* in, int N, int H, int W, int C, int in_ps, void* out, int out_ps, int dt,
                         hipStream_t s);

// out = x + x*g[n,c] (two roundings) [+ upper[y/2, x/2]], written as
// rep x rep blocks (rep = 1: plain) into a tensor of pixel stride out_ps.
void launch_gate_residual(const void* in, int N, int H, int W, int C, int in_ps, const float* gate,
                          const void* upper, int up_ps, void* out, int out_ps, int rep, int dt, hipStream_t s);
// Up to four gate_residual writes without an upper level (same N and
// storage type) in one launch: part i takes blocks first[i] .. first[i+1]-1.
struct GateResidualPart {
  const void* in;
  int H, W, C, in_ps;
  const float* gate;
  void* out;
  int out_ps, rep;
};
struct GateResidualMulti {
  GateResidualPart part[4];
  int count, N, dt;
};
void launch_gate_residual_multi(const GateResidualMulti& m, hipStream_t s);

// out[n, p, c] = x[n, p, c] * gate[n, c] rounded to the storage type; out is
// packed (pixel stride C).
void launch_scale_channels(const void* in, int N, int HW, int C, int in_ps, const float* gate, void* out, int dt,
                           hipStream_t s);

// Average pool, kernel [3,2], stride [3,2], count_include_pad = false.
void launch_avgpool32(const void* in, int N, int H, int W, int C, int in_ps, void* out, int Ho, int Wo, int dt,
                      hipStream_t s);

// Fused detector head tail: 2x2 s2 deconv (+bias, ReLU) then 2x2 s2 deconv to
// one channel (+bias) and sigmoid; in [N, H, W, Ch] -> fp32 out [N, 4H, 4W].
void launch_db_head_up(const void* in, int N, int H, int W, int Ch, int in_ps, const float* wu, const float* bu,
                       const float* wf, float bf, float* out, int dt, hipStream_t s);

// Row LayerNorm over C (eps), optional residual added after: out = LN(x) + r.
void launch_layer_norm(const void* in, int rows, int C, const float* w, const float* b, float eps, const void* res,
                       void* out, int dt, hipStream_t s);

// Multi-head attention core on qkv [B, T, 3*hidden] -> ctx [B, T, hidden].
// Register tile of the attention kernel for head dimension hd (0: too wide).
int attention_head_tile(int hd);
void launch_attention(const void* qkv, int B, int T, int hidden, int heads, void* out, int dt, hipStream_t s);

// In-place fp32 row softmax over `cols` columns.
void launch_softmax_rows(float* x, long rows, int cols, hipStream_t s);

// DB postprocess over N probability maps [N][H][W] (pixel index
// n*H*W + y*W + x < 2^31).  Work arrays: label/slot per pixel; per
// component slot (at most max_comp): count, root, keep, moments [6] (fp64),
// geom [8], extent [4]; out [max_comp][12] = polygon (8), score, image and
// root pixel (int bits), pad.  counters[0] = components, counters[1] =
// detections written.
struct DbParams {
  const float* prob;
  int N, H, W;
  long total;
  const int* content;        // [N][2] region examined: min(content, map) width, height
  const int* source;         // [N][2] source image width, height
  const int* content_scale;  // [N][2] content width, height of the transform
  float threshold, box_threshold, unclip;
  int min_area;
  int max_comp;
  int* label;
  int* slot;
  int* counters;
  int* count;
  int* root;
  int* keep;
  double* moments;
  float* geom;
  int* extent;
  float* out;
};
// The postprocess's kernels in launch order.  With `marks` (kDbKernels + 1
// events) an event is recorded before each kernel and after the last.
constexpr int kDbKernels = 8;
extern const char* const kDbKernelNames[kDbKernels];
void launch_db_postprocess(const DbParams& p, hipStream_t s, hipEvent_t* marks = nullptr);

// Static device scratch of the no-allocation postprocess entry point
// (db_scratch_bytes() bytes per device, held until the process ends).
// db_scratch looks its address up once per device (with that device made
// current for the lookup) and returns the cached address afterwards.
// db_scratch_mutex(device) serialises every use of one device's scratch
// (null for a device index outside [0, 64)).
size_t db_scratch_bytes();
hipError_t db_scratch(int device, void** ptr);
std::mutex* db_scratch_mutex(int device);

// Quad-bilinear RGB8 sampling -> rounded -> normalised NCHW fp32 planes.  One
// geometry per image: corners [N][8], content widths [N].
struct PreParams {
  const uint32_t* rgb;  // packed RGB8 bytes, 4-byte aligned
  int sw, sh;
  const float* corners;
  const int* content_w;
  int N, cw, ch;
  float scale[3], bias[3];
  float* out;     // fp32 NCHW planes [N][3][ch][cw], or
  void* nhwc4;    // (when set) the model input [N][ch][cw][4] in type `dt`, channel 3 zero
  int dt;
};
void launch_preprocess(const PreParams& p, hipStream_t s);

}  // namespace ppocr
