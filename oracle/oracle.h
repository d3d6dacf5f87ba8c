/*
 * CPU oracle for the FP16 conv-graph path — TEST INFRASTRUCTURE ONLY.
 *
 * A restatement of the reference CPU backend (backends/cpu) used as the
 * parity checker for the HIP backend and as the CPU baseline timed by
 * bench.py. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it. Nothing in the product links or calls it.
 *
 * All buffers are host memory. FP16 values are raw binary16 bit patterns.
 * Graph-level tensors are NCHW at this interface (the oracle re-lays them
 * to NHWC internally exactly like the reference plan); kernel-level entry
 * points take the NHWC buffers and packed weights the reference kernels
 * take. Every function returns 0 on success and -1 on error, with the
 * message available from oracle_last_error().
 */
#ifndef MLVC_ORACLE_H
#define MLVC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char* oracle_last_error(void);

/* ISA selector: 0 = AVX2+FMA+F16C path (reference default on x86),
 * 1 = scalar path (reference MLVC_CPU_ISA=scalar),
 * 2 = not a reference path: the AVX2 plan with every groups == 1 conv summed
 *     in the GPU kernels' order (16-channel steps, taps inside, each group of
 *     16 products added to the FP32 accumulator with one rounding). Used
 *     only to measure the effect of summation order alone. */

/* ---- graph level: CpuExecutionPlan (execution_plan.cpp:241-254) ---- */
/* bindings: n_bindings pairs (graph input index, graph output index). */
void* oracle_load(const char* model_dir, const char* model_name, const int64_t* bindings,
                  int n_bindings, int num_threads, int isa, int enable_fusion);
void oracle_free(void* plan);
int oracle_reset_state(void* plan);
int oracle_thread_count(void* plan);
int oracle_step_count(void* plan);
/* Counts and shapes of external inputs / outputs (bound state removed). */
int oracle_io_count(void* plan, int is_output);
int oracle_io_shape(void* plan, int is_output, int index, int64_t* shape4, int* rank);
int oracle_run(void* plan, const uint16_t* const* inputs, uint16_t* const* outputs);

/* ---- kernel level (NHWC buffers, reference kernel signatures) ---- */
int oracle_pack_conv(const uint16_t* w_oihw, const uint16_t* bias, int oc, int ic, int kh, int kw,
                     uint16_t* packed, size_t packed_elems);
size_t oracle_packed_conv_elems(int oc, int ic, int kh, int kw);
int oracle_pack_depthwise(const uint16_t* w_c1hw, const uint16_t* bias, int c, int kh, int kw,
                          uint16_t* packed, size_t packed_elems);
size_t oracle_packed_depthwise_elems(int c, int kh, int kw);
/* epi: 0 none, 1 clamp, 2 leaky relu, 3 residual add (residual NHWC [m, n]). */
int oracle_gemm_nhwc(size_t m, size_t n, size_t k, const uint16_t* lhs, const uint16_t* packed,
                     uint16_t* dst, int epi, float alpha, float cmin, float cmax,
                     const uint16_t* residual, int isa, int threads);
int oracle_spatial_conv_nhwc(const uint16_t* input, const uint16_t* packed, uint16_t* output, int n,
                             int ic, int ih, int iw, int oc, int oh, int ow, int kh, int kw, int sh,
                             int sw, int ph, int pw, int epi, float alpha, const uint16_t* residual,
                             int isa, int threads);
int oracle_depthwise_nhwc(const uint16_t* input, const uint16_t* packed, uint16_t* output, int n,
                          int c, int ih, int iw, int oh, int ow, int kh, int kw, int sh, int sw,
                          int ph, int pw, int isa, int threads);
int oracle_leaky_relu(const uint16_t* in, uint16_t* out, size_t count, float alpha, int isa);
int oracle_add(const uint16_t* a, const uint16_t* b, uint16_t* out, size_t count, int isa);
int oracle_depth_to_space_nhwc(const uint16_t* in, uint16_t* out, int n, int c, int h, int w, int block);
int oracle_space_to_depth_nhwc(const uint16_t* in, uint16_t* out, int n, int c, int h, int w, int block);
int oracle_nchw_to_nhwc(const uint16_t* in, uint16_t* out, size_t n, size_t c, size_t hw);
int oracle_nhwc_to_nchw(const uint16_t* in, uint16_t* out, size_t n, size_t hw, size_t c);
/* isa-2 model of one v_mfma_f32_32x32x16_f16 step for one output:
 * out[i] = c[i] + sum_k a[16i+k] * b[16i+k] as the matrix core sums it
 * (FP16 a, b as raw binary16; FP32 c and out), for count cases. */
int oracle_mfma_step(const uint16_t* a, const uint16_t* b, const float* c, float* out, size_t count);
/* Codec I/O: I420 frame (w x h) <-> model image [3, mh, mw] FP16.
 * pad5 = {left, right, top, bottom, rotated}. */
int oracle_yuv420_to_model(const uint8_t* yuv, int w, int h, int mw, int mh, int rotated, float pixel_range,
                           uint16_t* out);
int oracle_model_to_yuv420(const uint16_t* x, int w, int h, int mw, int mh, int pad_left, int pad_top, int rotated,
                           float pixel_range, uint8_t* yuv);
int oracle_frame_padding(int w, int h, int mw, int mh, int* pad5);
/* Operators of the real-model graphs (NHWC buffers as in the reference).
 * unary op: 0 clip [lo, hi], 1 sigmoid, 2 reciprocal, 3 round.
 * binary op: 0 add, 1 sub, 2 mul; the full dispatch of the reference plan
 * (same shape, scalar, channel and general broadcast). */
int oracle_unary(const uint16_t* in, uint16_t* out, size_t count, int op, float lo, float hi, int isa);
int oracle_binary(const uint16_t* a, const int64_t* a_shape, int a_rank, const uint16_t* b, const int64_t* b_shape, int b_rank,
                  uint16_t* out, const int64_t* out_shape, int out_rank, int op);
int oracle_slice_nhwc(const uint16_t* in, uint16_t* out, const int* id4, const int* od4, const int* starts, const int* steps);
/* dims4: n rows of logical NCHW dims. */
int oracle_concat_nhwc(const uint16_t* const* ins, const int* dims4, int n, uint16_t* out, const int* od4, int axis);
int oracle_gather(const uint16_t* data, const int64_t* shape, int rank, const int32_t* idx32, const int64_t* idx64, size_t count,
                  int axis, uint16_t* out);
int oracle_reglu_nhwc(const uint16_t* in, uint16_t* out, size_t spatial, size_t gate_channels, float lo, float hi, int isa);
/* scaled_out / blended_out may be NULL (the one-output form). */
int oracle_feature_update_nhwc(const uint16_t* in, const uint16_t* history, const uint16_t* scale, uint16_t* scaled_out,
                               uint16_t* blended_out, uint16_t* feature_out, size_t spatial, size_t channels, int isa);
int oracle_y0_tail_nhwc(const uint16_t* latent, const uint16_t* prior, const uint16_t* quant_scale, const uint16_t* us0,
                        const uint16_t* us1, uint16_t* normalized, uint16_t* clipped, uint16_t* y_raw, uint16_t* concat2,
                        uint16_t* concat3, float clip_min, size_t spatial, size_t q, int isa);
int oracle_y1_tail_nhwc(const uint16_t* normalized, const uint16_t* prior, const uint16_t* quant_scale, const uint16_t* us0,
                        const uint16_t* us1, const uint16_t* concat2, const uint16_t* clipped, uint16_t* y_raw, uint16_t* out,
                        size_t spatial, size_t q);
uint16_t oracle_float_to_half(float f);
float oracle_half_to_float(uint16_t h);

#ifdef __cplusplus
}
#endif
#endif
