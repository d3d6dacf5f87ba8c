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
int mlvc_backend_run(mlvc_backend* backend, const uint16_t* const* inputs, uint16_t* const* outputs);
/* InferenceBackend::reset_state() */
int mlvc_backend_reset_state(mlvc_backend* backend);
/* Names of the registered backends, comma-separated (available_backends()). */
int mlvc_backend_available(char* buf, size_t len);

/* ---- "hip" backend extras for measurement (no reference counterpart:
 *      the reference times whole run() calls only) ---- */
/* Uploads external inputs once; later frames reuse them in HBM. */
int mlvc_hip_backend_upload_inputs(mlvc_backend* backend, const uint16_t* const* inputs);
/* Replays `frames` per-frame hipGraphs back to back (device-resident, no
 * host copies) and returns the elapsed GPU time between events recorded on
 * the backend's stream around them. */
int mlvc_hip_backend_time_frames(mlvc_backend* backend, int frames, float* ms);
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

/* aot::load_aot_graph(model_dir, model_name) (runtime/src/aot_graph.cpp:
 * 291-317 with decode_graph's validation, :110-284) without any device
 * work: reports node/tensor counts and arena/weight sizes, or -1 with the
 * rejection message. */
int mlvc_aot_inspect(const char* model_dir, const char* model_name, int* nodes, int* tensors,
                     uint64_t* arena_bytes, uint64_t* weights_bytes);

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
