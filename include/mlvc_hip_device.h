/*
 * Thin device C ABI of the MI355X (gfx950) backend: memory, streams,
 * events, hipGraph capture and the hand-written HIP kernels of the FP16
 * conv-graph path.
 *
 * Plain C, POD arguments, opaque handles; the C++20 host never includes a
 * HIP header. This is the counterpart of the reference driver backend's
 * device boundary: the Driver-API wrapper (backends/driver_cubin/src/
 * driver.cpp:10-490, include/mlvc/driver_cubin/driver.hpp:145-190, handles
 * isolated in include/mlvc/driver_cubin/abi.hpp:1-34) and its
 * `extern "C" __global__` kernels launched by cuLaunchKernel
 * (driver.cpp:420-434). Each kernel entry point names the reference kernel
 * whose role it takes.
 *
 * All tensors are FP16 (raw binary16), channel-first NCHW, N = 1..n.
 * Every function returns 0 on success and -1 on failure; the message is
 * available from mlvc_hip_last_error() on the calling thread.
 */
#ifndef MLVC_HIP_DEVICE_H
#define MLVC_HIP_DEVICE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mlvc_hip_stream_s* mlvc_hip_stream;  /* hipStream_t */
typedef struct mlvc_hip_event_s* mlvc_hip_event;    /* hipEvent_t */
typedef struct mlvc_hip_graph_s* mlvc_hip_graph;    /* hipGraphExec_t */

const char* mlvc_hip_last_error(void);

/* ---- device, memory, streams (driver.cpp:10-140 DriverState/buffers) ---- */
int mlvc_hip_device_count(int* count);
int mlvc_hip_set_device(int device);
int mlvc_hip_device_name(int device, char* buf, size_t len);
int mlvc_hip_malloc(void** ptr, size_t bytes);
int mlvc_hip_free(void* ptr);
int mlvc_hip_host_alloc(void** ptr, size_t bytes); /* pinned */
int mlvc_hip_host_free(void* ptr);
int mlvc_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, mlvc_hip_stream s);
int mlvc_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, mlvc_hip_stream s);
int mlvc_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, mlvc_hip_stream s);
int mlvc_hip_stream_create(mlvc_hip_stream* s);
int mlvc_hip_stream_destroy(mlvc_hip_stream s);
int mlvc_hip_stream_synchronize(mlvc_hip_stream s);
int mlvc_hip_event_create(mlvc_hip_event* e);
int mlvc_hip_event_destroy(mlvc_hip_event e);
int mlvc_hip_event_record(mlvc_hip_event e, mlvc_hip_stream s);
int mlvc_hip_event_synchronize(mlvc_hip_event e);
int mlvc_hip_event_elapsed_ms(mlvc_hip_event start, mlvc_hip_event stop, float* ms);

/* ---- hipGraph capture/replay (driver.cpp:452-489 begin_capture/
 *      end_capture/launch_graph; cuda_graph_executor.cpp:38-52) ---- */
int mlvc_hip_capture_begin(mlvc_hip_stream s);
int mlvc_hip_capture_end(mlvc_hip_stream s, mlvc_hip_graph* graph);
int mlvc_hip_graph_launch(mlvc_hip_graph graph, mlvc_hip_stream s);
int mlvc_hip_graph_destroy(mlvc_hip_graph graph);

/* ---- convolution (groups == 1): MFMA implicit GEMM ----
 * Replaces the reference's 1x1 GEMM kernels (pointwise_conv.cu:116-338,
 * cutlass.cu:116-143), implicit-GEMM KxK convs (spatial_conv.cu:1-293,
 * cutlass.cu:145-161 with its layout.cu:1-48 NCHW<->NHWC transposes) and
 * the generic fallback (generic_conv.cu:1-82). Semantics follow
 * backends/cpu: y = fp16(bias + sum x*w) with FP32 accumulation, then the
 * epilogue on the rounded value (kernels_scalar.cpp:160-195).
 *
 * Fusions (all optional):
 *   in_s2d_block > 1 : the conv input is SPACE_TO_DEPTH(block) of `x`, read
 *                      through the CRD index map (x is [n, ic/b^2, ih*b, iw*b]);
 *   x2 != NULL       : the conv input is the channel CONCAT of `x`
 *                      (channels [0, ic_split)) and `x2` (the rest);
 *   epilogue         : LeakyReLU(alpha) or residual ADD of `residual`;
 *   out_d2s_block > 1: the output is written through DEPTH_TO_SPACE(block)
 *                      (CRD), y is [n, oc/b^2, oh*b, ow*b].
 */
enum { MLVC_EPI_NONE = 0, MLVC_EPI_LEAKY_RELU = 1, MLVC_EPI_RESIDUAL_ADD = 2, MLVC_EPI_REGLU = 3, MLVC_EPI_CLAMP = 4 };
/* MLVC_EPI_CLAMP (the reference's GEMM kClamp epilogue, fusion_matcher.cpp:
 * 378-389, kernels_x86_avx2.cpp:196-198): y = max(min(fp16(acc), clip_hi),
 * clip_lo), NaN giving clip_hi as in the vector lanes. */
/* MLVC_EPI_REGLU (the reference's 1x1 conv with a ReGLU epilogue,
 * backends/cpu/src/fusion_matcher.cpp:258-302): the conv computes oc = 2G
 * channels, rounded to FP16, and writes y [n, G, oh, ow] =
 * fp16(fp16(clip(gate, clip_lo, clip_hi)) * linear). The weight and bias rows
 * are given in blocks of 64: 32 gate rows g..g+31 followed by the 32 linear
 * rows G+g..G+g+31 (g = 32 * block), so G must be a multiple of 32; no
 * DEPTH_TO_SPACE output. */

typedef struct mlvc_hip_conv_desc {
    int n, ic, ih, iw;                 /* conv input geometry (after fusion maps) */
    int oc, oh, ow;                    /* conv output geometry (before d2s) */
    int kh, kw, stride_h, stride_w, pad_h, pad_w;
    const void* x;
    const void* x2;
    int ic_split;
    int in_s2d_block;
    const void* packed_w;              /* from mlvc_hip_conv_pack */
    const float* bias;                 /* fp32 widening of the fp16 bias, length mlvc_hip_conv_bias_len */
    int epilogue;
    float alpha;
    float clip_lo, clip_hi;            /* MLVC_EPI_CLAMP / MLVC_EPI_REGLU bounds */
    const void* residual;              /* [n, oc, oh, ow] */
    void* y;
    int out_d2s_block;
    int variant;                       /* tile configuration; set by mlvc_hip_conv_plan */
    int vector_io;                     /* 16-byte row staging eligible; set by mlvc_hip_conv_plan */
    int ksplit, split_c;               /* split K; set by mlvc_hip_conv_plan (below) */
    void* workspace;                   /* FP32 partials of a split conv, mlvc_hip_conv_workspace_bytes */
    size_t workspace_bytes;
    /* Channel-last x ([n, ih, iw, ic]) / y ([n, oh, ow, oc]): set by the
     * backend where a conv hands its activations to or from a fused
     * residual block (no counterpart in the reference, whose tensors are
     * NCHW at every node boundary). 3x3 weight-streaming variants only;
     * channel counts a multiple of 8; in: no concat or space_to_depth
     * fusion; out: LeakyReLU, clamp or no epilogue, and with
     * depth_to_space(2) a multiple of 8 output channels after it
     * (y: [n, 2 oh, 2 ow, oc / 4]). */
    int in_nhwc, out_nhwc;
} mlvc_hip_conv_desc;

/* Chooses the kernel variant for the geometry by a cost model (sets
 * desc->variant and desc->vector_io). Every 3x3 variant accumulates in the
 * same K order, and so does every 1x1 variant, so the choice never changes
 * results. Role of the reference's per-shape tile choice by fixed thresholds
 * (backends/driver_cubin/src/execution_plan.cpp:151-181, 374-432).
 *
 * Also sets the split K of the geometry (a fixed rule of the conv geometry
 * alone, independent of the variant, the epilogue and the fusions, so it
 * never depends on tuning and fused and unfused schedules agree): a 1x1
 * conv with K = ic >= 576 (above the 512-channel projections of the fused
 * residual block, which are not split) and fewer than 512 work items of 128
 * output channels x 128 pixels (items = n * ceil(oc/128) * ceil(oh*ow/128))
 * is split into ksplit =
 * ceil(ic / split_c) ranges of input channels, split_c = 64 * ceil(ic /
 * (64 * s)), s = min(8, 512 / items, ic / 64) (integer division; no split
 * when s <= 1). Split s sums its channels in the usual K order into an FP32
 * partial (split 0 seeded with the bias, the others with zero); a second
 * kernel adds the partials in split order, rounds to FP16 and applies the
 * epilogue (ReGLU included) and the DEPTH_TO_SPACE store. Split convs run on
 * the conv_mfma variants only and need desc->workspace (FP32 partials,
 * mlvc_hip_conv_workspace_bytes; 16-byte aligned). The reference's role for
 * this: its small-tile choice where a large-tile grid would be under two
 * waves of SMs (driver_cubin/src/execution_plan.cpp:379-391). */
int mlvc_hip_conv_plan(mlvc_hip_conv_desc* desc);
/* Bytes of FP32 partials a launch of desc needs (0 when not split). */
size_t mlvc_hip_conv_workspace_bytes(const mlvc_hip_conv_desc* desc);
/* Lists every variant that can run the geometry (for measuring them on the
 * device and keeping the fastest); *count receives the total. */
int mlvc_hip_conv_candidates(const mlvc_hip_conv_desc* desc, int* variants, int capacity, int* count);
const char* mlvc_hip_conv_variant_name(int variant);
size_t mlvc_hip_conv_packed_bytes(const mlvc_hip_conv_desc* desc);
size_t mlvc_hip_conv_bias_len(const mlvc_hip_conv_desc* desc);
/* Host-side repack of OIHW fp16 weights into the variant's MFMA fragment
 * order (reference role: pack_conv_weights_f16p16x1bias,
 * kernels_scalar.cpp:14-56, and mlvc_oihw_to_krsc_fp16, layout.cu). */
int mlvc_hip_conv_pack(const mlvc_hip_conv_desc* desc, const uint16_t* w_oihw, void* dst_host);
int mlvc_hip_conv_launch(const mlvc_hip_conv_desc* desc, mlvc_hip_stream s);
/* mlvc_hip_conv_launch without a caller workspace, allocating nothing: a
 * split-K conv keeps its FP32 partials in a static device array of the
 * library (32 MiB, one per GPU, held until the process ends) instead of
 * desc->workspace, which is ignored. Every split mlvc_hip_conv_plan chooses
 * fits (its partials are at most 512 x 128 x 128 FP32 values); a larger one
 * set by hand fails with an error before anything is launched. Each call
 * overwrites every partial it reads, so nothing needs clearing between
 * calls; calls that overlap on one GPU (on different streams) share the
 * array and race. No counterpart in the reference: for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). */
int mlvc_hip_conv_launch_noalloc(const mlvc_hip_conv_desc* desc, mlvc_hip_stream s);

/* ---- depthwise KxK (groups == C == OC) ----
 * Replaces mlvc_depthwise_conv_fp16{,_pair,_quad} (depthwise_conv.cu:1-173);
 * semantics of backends/cpu avx2_depthwise3x3_s1p1 (kernels_x86_avx2.cpp:
 * 237-302): FP32 accumulator seeded with the bias, taps in (ky,kx) order,
 * out-of-range taps skipped. `w` is [c, 1, kh, kw] fp16, `bias` fp32 [c]. */
int mlvc_hip_depthwise(const void* x, const uint16_t* w, const float* bias, void* y, int n, int c,
                       int ih, int iw, int oh, int ow, int kh, int kw, int stride_h, int stride_w,
                       int pad_h, int pad_w, mlvc_hip_stream s);

/* ---- fused depthwise-separable residual block ----
 * y = fp16(fp16(W2 e + b2) + x), e = fp16(LeakyReLU(fp16(W1 d + b1))),
 * d = fp16(DW3x3(x) + b0): one kernel for the DW conv (depthwise_conv.cu),
 * the 1x1 expand with LeakyReLU epilogue and the 1x1 project with residual
 * epilogue (pointwise_conv.cu / cutlass.cu EVT epilogues) that the
 * reference runs as three launches; rounding points are unchanged.
 * x, y: [n, c, h, w] (or channel-last, below); dw_w: [c, 1, 3, 3] fp16 (stride 1, pad 1);
 * w1: W1 [e, c] packed by mlvc_hip_dwblock_pack; w2: W2 [c, e] packed.
 * x, y and dw_w must be 16-byte aligned. */
typedef struct mlvc_hip_dwblock_desc {
    int n, c, e, h, w;
    const void* x;
    void* y;
    const uint16_t* dw_w;
    const float* dw_b;
    const void* w1;
    const float* b1;
    const void* w2;
    const float* b2;
    float alpha;
    /* Layouts of x and y: 0 = NCHW, 1 = channel-last [n, h, w, c]. The
     * backend sets them for a block whose output feeds only the next block
     * (no counterpart in the reference, whose tensors are NCHW at every
     * node boundary; here the handover between chained blocks is internal).
     * x and y must not alias. */
    int in_nhwc, out_nhwc;
} mlvc_hip_dwblock_desc;

/* 1 when (c, e, h, w) has a fused-block kernel, else 0. */
int mlvc_hip_dwblock_supported(int c, int e, int h, int w);
size_t mlvc_hip_dwblock_packed_bytes(int m, int k);
/* Host-side repack of a row-major [m, k] fp16 matrix into MFMA A-fragment order. */
int mlvc_hip_dwblock_pack(const uint16_t* w_mk, int m, int k, void* dst_host);
int mlvc_hip_dwblock_launch(const mlvc_hip_dwblock_desc* desc, mlvc_hip_stream s);

/* ---- fused conv pair: 3x3 conv -> channel CONCAT -> 1x1 conv ----
 * y = epi_b(fp16(Wb [t ; r] + bb)),  t = epi_a(fp16(Wa * x + ba))
 * with t never leaving the chip: one kernel for what the reference runs as a
 * spatial conv (spatial_conv.cu / cutlass.cu fprop), a channel concat
 * (tensor_ops.cu concat copy) and a 1x1 conv (pointwise_conv.cu), or the
 * CPU plan's two GEMM steps (execution_plan.cpp); rounding points and K
 * order are those of the unfused kernels, so the results are identical.
 * x: [n, ica, h, w], or with in_s2d_block == 2 the SPACE_TO_DEPTH source
 * [n, ica/4, 2h, 2w]; r: [n, cr, h, w]; y: [n, ocb, h, w]. Wa is OIHW
 * [oca, ica, 3, 3] (stride 1, pad 1), Wb is [ocb, oca + cr]; both packed
 * by mlvc_hip_convpair_pack. Biases are FP32. */
typedef struct mlvc_hip_convpair_desc {
    int n, ica, h, w, in_s2d_block;
    int oca, cr, ocb;
    const void* x;
    const void* r;
    const void* wa;
    const float* ba;
    int epi_a;
    float alpha_a;
    const void* wb;
    const float* bb;
    int epi_b;
    float alpha_b;
    void* y;
} mlvc_hip_convpair_desc;

/* 1 when the geometry has a fused kernel (oca = cr = ocb = 64, w % 8 == 0,
 * epilogues none or LeakyReLU), else 0. */
int mlvc_hip_convpair_supported(const mlvc_hip_convpair_desc* desc);
size_t mlvc_hip_convpair_packed_a_bytes(const mlvc_hip_convpair_desc* desc);
size_t mlvc_hip_convpair_packed_b_bytes(const mlvc_hip_convpair_desc* desc);
int mlvc_hip_convpair_pack(const mlvc_hip_convpair_desc* desc, const uint16_t* wa_oihw, const uint16_t* wb_oi,
                           void* dst_a_host, void* dst_b_host);
int mlvc_hip_convpair_launch(const mlvc_hip_convpair_desc* desc, mlvc_hip_stream s);

/* ---- pixel layout, CRD (tensor_ops.cu:62-116, mode 1) ----
 * DEPTH_TO_SPACE: in [n, c*b*b, h, w] -> out [n, c, h*b, w*b].
 * SPACE_TO_DEPTH: in [n, c, h, w] -> out [n, c*b*b, h/b, w/b]. */
int mlvc_hip_depth_to_space(const void* x, void* y, int n, int in_c, int h, int w, int block, mlvc_hip_stream s);
int mlvc_hip_space_to_depth(const void* x, void* y, int n, int in_c, int h, int w, int block, mlvc_hip_stream s);

/* ---- elementwise (elementwise.cu:1-80): y = fp16(op(fp32 inputs)) ---- */
int mlvc_hip_leaky_relu(const void* x, void* y, size_t count, float alpha, mlvc_hip_stream s);

/* ---- Codec I/O around the encoder / decoder graphs ----
 * Frames are I420 bytes (Y w*h, then U and V (w/2)*(h/2)); the model image
 * is FP16 [3, mh, mw]. Replace the driver backend's mlvc_yuv420_to_nchw_fp16
 * and mlvc_nchw_to_yuv420 (backends/driver_cubin/kernels/codec_io.cu:31-107)
 * with the CPU backend's values (backends/cpu/src/execution_plan.cpp:
 * 1044-1322): lut holds 256 FP16 values float_to_half(v / 255 * pixel_range)
 * in device memory; the frame sits at model (0, 0) with its last column/row
 * repeated, transposed when rotated. The model -> frame direction reads the
 * active area at (pad_top, pad_left), divides by pixel_range, averages chroma
 * over 2x2 and rounds v * 255 half to even after clamping to [0, 1]. */
int mlvc_hip_yuv420_to_model(const uint8_t* yuv, const uint16_t* lut, void* out, int w, int h, int mw, int mh,
                             int rotated, mlvc_hip_stream s);
int mlvc_hip_model_to_yuv420(const void* x, uint8_t* yuv, int w, int h, int mw, int mh, int pad_left, int pad_top,
                             int rotated, float pixel_range, mlvc_hip_stream s);
int mlvc_hip_add(const void* a, const void* b, void* y, size_t count, mlvc_hip_stream s);
/* Channel concat of two NCHW tensors (tensor_ops.cu concat copy, axis 1). */
int mlvc_hip_concat_channels(const void* a, int ca, const void* b, int cb, void* y, int n, size_t hw,
                             mlvc_hip_stream s);
/* Zero fill by kernel (safe inside captured graphs). */
int mlvc_hip_zero(void* y, size_t bytes, mlvc_hip_stream s);
/* Fills bytes / 2 FP16 values in [-1, 1), |v| >= 0.5, from a hash of the
 * element index and seed (deterministic); for timing kernels on data that
 * loads the matrix cores like real activations. */
int mlvc_hip_fill_pattern(void* y, size_t bytes, unsigned seed, mlvc_hip_stream s);

/* ---- operators of the real MLVC graphs (NCHW FP16) ----
 * Same values as the reference CPU kernels (backends/cpu/src/
 * kernels_scalar.cpp:80-110, 244-537; kernels_x86_avx2.cpp:30-62, 304-712)
 * computed per element in FP32 with one RNE rounding per materialised value;
 * the driver backend's counterparts are kernels/elementwise.cu,
 * tensor_ops.cu, activation.cu, recurrent_feature.cu and
 * quantization_tail.cu. Buffers of the vector paths are 16-byte aligned. */
enum { MLVC_UNARY_CLIP = 0, MLVC_UNARY_SIGMOID = 1, MLVC_UNARY_RECIPROCAL = 2, MLVC_UNARY_ROUND = 3 };
/* CLIP to [lo, hi] (NaN -> hi, as the reference's vector lanes), SIGMOID
 * with the reference's vector exponential, 1/x, round half to even. */
int mlvc_hip_unary(const void* x, void* y, size_t count, int op, float lo, float hi, mlvc_hip_stream s);
enum { MLVC_BINARY_ADD = 0, MLVC_BINARY_SUB = 1, MLVC_BINARY_MUL = 2 };
/* y = a op b on right-aligned 4-D dims; an operand dim of 1 broadcasts. */
int mlvc_hip_binary(const void* a, const int64_t* a_dims, const void* b, const int64_t* b_dims, void* y,
                    const int64_t* y_dims, int op, mlvc_hip_stream s);
/* y[i] = x[starts + i * steps] per dim (4-D); every read must lie in x. */
int mlvc_hip_slice(const void* x, const int64_t* x_dims, void* y, const int64_t* y_dims, const int64_t* starts,
                   const int64_t* steps, mlvc_hip_stream s);
/* rows x row_elems block copy between row strides (a CONCAT input placed
 * into its output). */
int mlvc_hip_copy_rows(const void* x, void* y, size_t rows, size_t row_elems, size_t x_stride, size_t y_stride,
                       mlvc_hip_stream s);
/* y[o][i][r] = data[o][indices[i]][r] for data viewed as [outer, axis_dim,
 * inner]; indices int32 or int64 in device memory, negative ones count from
 * the end; the caller checks the range (the kernel clamps). */
int mlvc_hip_gather(const void* data, const void* indices, int indices_int64, size_t count, size_t outer,
                    size_t axis_dim, size_t inner, void* y, mlvc_hip_stream s);
/* x [n, 2G, hw] -> y [n, G, hw] = fp16(fp16(clamp(gate, lo, hi)) * linear)
 * (reglu_nhwc, kernels_scalar.cpp:304-322). */
int mlvc_hip_reglu(const void* x, void* y, int n, int gate_channels, size_t hw, float lo, float hi, mlvc_hip_stream s);
/* Device tables used by the kernels below (the feature update's gate
 * table), computed once per device on stream s, which is waited for. No
 * counterpart in the reference (its kernels compute the gate directly).
 * Launchers prepare them on first use, except under graph capture, where
 * they fail: a caller that captures calls this first. */
int mlvc_hip_prepare_tables(mlvc_hip_stream s);

/* Recurrent feature update (feature_update[_outputs]_nhwc,
 * kernels_scalar.cpp:324-405): x [n, 3C, hw], history [n, C, hw], scale [C]
 * -> feature [n, 2C, hw] = scaled | blended; scaled / blended [n, C, hw]
 * also written when both are non-null. */
int mlvc_hip_feature_update(const void* x, const void* history, const void* scale, void* feature, void* scaled,
                            void* blended, int n, int channels, size_t hw, mlvc_hip_stream s);
/* y0 / y1 quantisation tails (kernels_scalar.cpp:407-537); planes of
 * [n, 2q, hw] unless noted: prior [n, 4q, hw] (y0) or [n, 2q, hw] (y1),
 * update scales and y_raw [n, q, hw], concat3 [n, 6q, hw]. */
typedef struct mlvc_hip_y0_tail_desc {
    const void* latent;
    const void* prior;
    const void* quant_scale;
    const void* update_scale0;
    const void* update_scale1;
    void* normalized;
    void* clipped;
    void* y_raw;
    void* concat2;
    void* concat3;
    int n, q;
    size_t hw;
    float clip_min;
} mlvc_hip_y0_tail_desc;
int mlvc_hip_y0_tail(const mlvc_hip_y0_tail_desc* desc, mlvc_hip_stream s);
typedef struct mlvc_hip_y1_tail_desc {
    const void* normalized;
    const void* prior;
    const void* quant_scale;
    const void* update_scale0;
    const void* update_scale1;
    const void* concat2;
    const void* clipped;
    void* y_raw;
    void* out;
    int n, q;
    size_t hw;
} mlvc_hip_y1_tail_desc;
int mlvc_hip_y1_tail(const mlvc_hip_y1_tail_desc* desc, mlvc_hip_stream s);

#ifdef __cplusplus
}
#endif
#endif
