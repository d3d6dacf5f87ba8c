/*
 * C ABI of the MI355X backend at the reference's plugin boundary.
 *
 * The reference exposes its inference backends as the C++ interface
 * mlvc::InferenceBackend (runtime/include/mlvc/runtime/backend.hpp:48-63:
 * name/load/run/reset_state) created through the named registry
 * (backend.hpp:98-110, runtime/src/backend_registry.cpp:83-113). This header
 * is the same boundary as plain C so that any FFI can bind it: each handle
 * wraps a backend created by mlvc::create_backend (the "hip" backend is
 * registered by this library), and errors follow the reference's public C
 * ABI convention (public/include/mlvc/codec.h:76-86, codec/src/c_api.cpp:
 * 71-88): -1 plus a NUL-terminated message, here from
 * mlvc_backend_last_error().
 *
 * Tensors cross the boundary as host buffers of raw binary16 in NCHW graph
 * order with bound state tensors removed, exactly as run() takes and
 * returns them (execution_plan.cpp:1623-1675).
 */
#ifndef MLVC_HIP_BACKEND_H
#define MLVC_HIP_BACKEND_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mlvc_backend mlvc_backend;

const char* mlvc_backend_last_error(void);

/* create_backend(BackendOptions{backend_name, model_dir, device_id,
 * num_threads}) — backend.hpp:24-32, 110. */
int mlvc_backend_create(const char* backend_name, const char* model_dir, int device_id, int num_threads,
                        mlvc_backend** out);
void mlvc_backend_destroy(mlvc_backend* backend);
/* InferenceBackend::name() */
const char* mlvc_backend_name(const mlvc_backend* backend);
/* InferenceBackend::load(model_name, ModelExecutionConfig); bindings holds
 * n_bindings (input_index, output_index) pairs of StateTensorBinding
 * (backend.hpp:34-46), dtype FP16, shape taken from the graph. */
int mlvc_backend_load(mlvc_backend* backend, const char* model_name, const int64_t* bindings, int n_bindings);
/* Number and NCHW shapes of run()'s external inputs / outputs. */
int mlvc_backend_io_count(mlvc_backend* backend, int is_output, int* count);
int mlvc_backend_io_shape(mlvc_backend* backend, int is_output, int index, int64_t* shape4, int* rank);
/* InferenceBackend::run(inputs) -> outputs (host buffers, sizes implied by
 * the shapes above). */
int mlvc_backend_run(mlvc_backend* backend, const void* const* inputs, uint16_t* const* outputs);
/* Element type of external input/output `index`: 0 FP16, 1 INT32 (control
 * inputs such as q_index_shifted; outputs are FP16). */
int mlvc_backend_io_dtype(mlvc_backend* backend, int is_output, int index, int* dtype);
/* InferenceBackend::reset_state() */
int mlvc_backend_reset_state(mlvc_backend* backend);
/* Names of the registered backends, comma-separated (available_backends()). */
int mlvc_backend_available(char* buf, size_t len);

/* ---- BufferedCodecBackend (backend.hpp:64-96), for backends that have it
 *      (-1 "backend has no buffered codec I/O" otherwise) ----
 * configure_codec_io(CodecIoConfig{width, height, model_width, model_height,
 * pixel_range, FramePadding{left, right, top, bottom, rotated}, slots}); the
 * graph must be MLVCEncoder or MLVCDecoder with an INT32 [1]
 * q_index_shifted input and an FP16 [1, 3, model_height, model_width] x
 * input (encoder) or x_hat output (decoder): backends/cpu/src/
 * execution_plan.cpp:1386-1486, backends/driver_cubin/src/
 * cuda_graph_executor.cpp:205-236. */
int mlvc_backend_configure_codec_io(mlvc_backend* backend, int width, int height, int model_width, int model_height,
                                    float pixel_range, int pad_left, int pad_right, int pad_top, int pad_bottom,
                                    int rotated, size_t slots);
int mlvc_backend_codec_slot_count(mlvc_backend* backend, size_t* count);
/* encoder_input_yuv(slot): the slot's pinned I420 planes, writable until the
 * slot is submitted (cuda_graph_executor.cpp:243-259). */
int mlvc_backend_encoder_input_yuv(mlvc_backend* backend, size_t slot, uint8_t** y, uint8_t** u, uint8_t** v);
/* submit_encoder(slot, shifted_q): frame upload, conversion, frame graph,
 * output download, in stream order (cuda_graph_executor.cpp:261-290). */
int mlvc_backend_submit_encoder(mlvc_backend* backend, size_t slot, int shifted_q);
/* encoder_outputs(slot)[index] / decoder_inputs(slot)[index]: pinned host
 * bytes of the external outputs / of the external inputs other than
 * q_index_shifted, in graph order (cuda_graph_executor.cpp:292-334). */
int mlvc_backend_codec_tensor_count(mlvc_backend* backend, size_t slot, int is_decoder, int* count);
int mlvc_backend_encoder_output(mlvc_backend* backend, size_t slot, int index, const void** data, size_t* bytes);
int mlvc_backend_decoder_input(mlvc_backend* backend, size_t slot, int index, void** data, size_t* bytes);
/* submit_decoder(slot, shifted_q): input uploads, frame graph, conversion,
 * frame download (cuda_graph_executor.cpp:336-373). */
int mlvc_backend_submit_decoder(mlvc_backend* backend, size_t slot, int shifted_q);
int mlvc_backend_decoder_output_yuv(mlvc_backend* backend, size_t slot, const uint8_t** y, const uint8_t** u,
                                    const uint8_t** v);
/* wait_codec_slot(slot) (cuda_graph_executor.cpp:393-400). A submitted slot
 * must be waited before its views are used again; touching it earlier
 * fails with "codec slot is pending". */
int mlvc_backend_wait_codec_slot(mlvc_backend* backend, size_t slot);
/* frame_padding(width, height, model_width, model_height) of core/src/
 * yuv.cpp:325-337: pad5 = {left, right, top, bottom, rotated}. */
int mlvc_frame_padding(int width, int height, int model_width, int model_height, int* pad5);

/* ---- "hip" backend extras for measurement (no reference counterpart:
 *      the reference times whole run() calls only) ---- */
/* Uploads external inputs once; later frames reuse them in HBM. */
int mlvc_hip_backend_upload_inputs(mlvc_backend* backend, const void* const* inputs);
/* Replays `frames` per-frame hipGraphs back to back (device-resident, no
 * host copies) and returns the elapsed GPU time between events recorded on
 * the backend's stream around them. */
int mlvc_hip_backend_time_frames(mlvc_backend* backend, int frames, float* ms);
/* The same replays with events recorded just before and after every frame:
 * ms_each[f] is frame f's GPU time (1 <= frames <= 4096). flush_bytes > 0
 * runs a device-to-device copy of flush_bytes / 2 bytes before each frame,
 * outside its events, so each frame starts with cold L2 and MALL. */
int mlvc_hip_backend_time_frames_each(mlvc_backend* backend, int frames, size_t flush_bytes, float* ms_each);
/* Copies the current external outputs to the host. */
int mlvc_hip_backend_download_outputs(mlvc_backend* backend, uint16_t* const* outputs);
/* Kernel launches of one frame. info: name, kernel variant, FLOPs and
 * algorithmic bytes (each tensor read or written once). */
int mlvc_hip_backend_launch_count(mlvc_backend* backend, int* count);
int mlvc_hip_backend_launch_info(mlvc_backend* backend, int index, char* name, size_t name_len, char* kind,
                                 size_t kind_len, double* flops, double* bytes);
/* Launches kernel `index` `reps` times back to back on the backend's stream
 * between two events and reports the mean duration per launch. */
int mlvc_hip_backend_time_launch(mlvc_backend* backend, int index, int reps, float* ms_per_launch);
/* Launches kernel `index` `reps` times, one at a time, each after a
 * device-to-device copy of flush_bytes / 2 bytes (outside its events) that
 * evicts L2 and the MALL, and writes each launch's duration to ms_each[reps]
 * (1 <= reps <= 4096). No counterpart in the reference: a measurement helper
 * beside mlvc_hip_backend_time_frames_each. */
int mlvc_hip_backend_time_launch_cold(mlvc_backend* backend, int index, int reps, size_t flush_bytes, float* ms_each);

/* aot::load_aot_graph(model_dir, model_name) (runtime/src/aot_graph.cpp:
 * 291-317 with decode_graph's validation, :110-284) without any device
 * work: reports node/tensor counts and arena/weight sizes, or -1 with the
 * rejection message. */
int mlvc_aot_inspect(const char* model_dir, const char* model_name, int* nodes, int* tensors,
                     uint64_t* arena_bytes, uint64_t* weights_bytes);

/* ---- bundle / asset path ----
 * Model directories or "embedded:<profile>" locations (reference
 * core/src/model_assets.cpp:36-252; the embedded image is described in
 * mlvc_embedded_models.h).
 * mlvc_model_config_json: load_model_config (core/src/model.cpp:150-183:
 * metadata.pb checked against model_bundle.pb, ModelConfig::validate,
 * :50-91) as a JSON object of the ModelConfig members plus the derived
 * feature / latent / hyperprior dimensions; -1 with the reference's message
 * on any mismatch. mlvc_model_verify_bundle: every artifact of model_bundle.pb
 * present with its recorded size and SHA-256 (the check of the reference's
 * packager, tools/python/mlvc_tools/package.py:97-145, done in C++). */
int mlvc_model_config_json(const char* model_dir, char* buf, size_t len);
int mlvc_model_verify_bundle(const char* model_dir);
/* model_bundle.pb of a location as JSON: profile, model_version, width,
 * height and the artifacts (path, size) it lists. */
int mlvc_model_bundle_json(const char* model_dir, char* buf, size_t len);
/* Profiles of the linked embedded model image, newline-separated, in index
 * order (list_embedded_model_profiles, model_assets.cpp:204-214); empty when
 * none is linked. */
int mlvc_model_embedded_profiles(char* buf, size_t len);
/* "embedded:mlvc-psnr-v1" when that profile is embedded, else the first
 * embedded profile, else "" (default_model_location, model_assets.cpp:
 * 216-225). */
int mlvc_model_default_location(char* buf, size_t len);

/* ---- seeded synthetic graphs (graph.pb / weights.bin / metadata.pb) ---- */
int mlvc_synth_configs(char* buf, size_t len);
int mlvc_synth_write(const char* config, const char* out_dir, uint64_t seed);
/* External input `index` of frame `frame`: count fp16 values. */
int mlvc_synth_input(const char* config, int index, int frame, uint64_t seed, uint16_t* dst, size_t count);
/* State bindings of the config (pairs) and its frame count. */
int mlvc_synth_bindings(const char* config, int64_t* pairs, int max_pairs, int* n_pairs, int* frames);

#ifdef __cplusplus
}
#endif
#endif
