// C ABI over mlvc::InferenceBackend (include/mlvc_hip_backend.h).
// Exceptions become -1 plus a per-thread message, as in the reference's
// codec/src/c_api.cpp:71-88.

#include "hip_backend.hpp"
#include "mlvc/runtime/graph_builder.hpp"
#include "mlvc_hip_backend.h"

#include "mlvc/core/assets.hpp"
#include "mlvc/core/model.hpp"
#include "mlvc/runtime/wire.hpp"

#include <cstring>
#include <optional>
#include <cstdio>
#include <filesystem>
#include <stdexcept>
#include <string>

struct mlvc_backend {
    std::unique_ptr<mlvc::InferenceBackend> impl;
    std::string name;
    std::string model_dir;
};

namespace {

thread_local std::string g_error;

template <typename F>
int guard(F&& fn)
{
    try {
        fn();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

mlvc::hip_backend::HipBackend& hip(mlvc_backend* b)
{
    auto* h = dynamic_cast<mlvc::hip_backend::HipBackend*>(b->impl.get());
    if (!h) throw std::runtime_error("not a hip backend: " + b->name);
    return *h;
}

// The buffered codec path, as the reference's callers find it
// (codec/src/pipeline.cpp:826, 906: dynamic_cast to BufferedCodecBackend).
mlvc::BufferedCodecBackend& buffered(mlvc_backend* b)
{
    auto* c = dynamic_cast<mlvc::BufferedCodecBackend*>(b->impl.get());
    if (!c) throw std::runtime_error(b->name + ": backend has no buffered codec I/O");
    return *c;
}

std::vector<std::vector<std::int64_t>> shapes(mlvc_backend* b, bool outputs)
{
    return hip(b).io_shapes(outputs);
}

void copy_str(const std::string& s, char* buf, std::size_t len)
{
    if (!buf || len == 0) return;
    const std::size_t n = std::min(len - 1, s.size());
    std::memcpy(buf, s.data(), n);
    buf[n] = '\0';
}

}  // namespace

extern "C" {

const char* mlvc_backend_last_error(void) { return g_error.c_str(); }

int mlvc_backend_create(const char* backend_name, const char* model_dir, int device_id, int num_threads, mlvc_backend** out)
{
    return guard([&] {
        mlvc::BackendOptions o;
        o.backend_name = backend_name ? backend_name : "";
        o.model_dir = model_dir ? model_dir : "";
        o.device_id = device_id;
        o.num_threads = num_threads;
        auto b = std::make_unique<mlvc_backend>();
        b->impl = mlvc::create_backend(o);
        b->name = std::string(b->impl->name());
        b->model_dir = o.model_dir;
        *out = b.release();
    });
}

void mlvc_backend_destroy(mlvc_backend* backend) { delete backend; }

const char* mlvc_backend_name(const mlvc_backend* backend) { return backend->name.c_str(); }

int mlvc_backend_load(mlvc_backend* backend, const char* model_name, const int64_t* bindings, int n_bindings)
{
    return guard([&] {
        // StateTensorBinding carries the bound tensor's shape; take it from
        // the graph's own input descriptor.
        mlvc::ModelExecutionConfig cfg;
        if (n_bindings > 0) {
            const auto g = mlvc::aot::load_aot_graph(std::filesystem::path(backend->model_dir), model_name);
            for (int i = 0; i < n_bindings; ++i) {
                mlvc::StateTensorBinding b;
                b.input_index = static_cast<std::size_t>(bindings[2 * i]);
                b.output_index = static_cast<std::size_t>(bindings[2 * i + 1]);
                if (b.input_index >= g.descriptor.inputs.size())
                    throw std::runtime_error("state binding index out of range");
                b.shape = g.descriptor.tensors[g.descriptor.inputs[b.input_index]].shape;
                cfg.state_bindings.push_back(b);
            }
        }
        backend->impl->load(model_name, cfg);
    });
}

int mlvc_backend_io_count(mlvc_backend* backend, int is_output, int* count)
{
    return guard([&] { *count = static_cast<int>(shapes(backend, is_output != 0).size()); });
}

int mlvc_backend_io_shape(mlvc_backend* backend, int is_output, int index, int64_t* shape4, int* rank)
{
    return guard([&] {
        const auto s = shapes(backend, is_output != 0).at(static_cast<std::size_t>(index));
        *rank = static_cast<int>(s.size());
        for (std::size_t i = 0; i < s.size() && i < 4; ++i) shape4[i] = s[i];
    });
}

int mlvc_backend_io_dtype(mlvc_backend* backend, int is_output, int index, int* dtype)
{
    return guard([&] {
        const auto t = hip(backend).io_dtypes(is_output != 0).at(static_cast<std::size_t>(index));
        *dtype = t == mlvc::TensorDataType::kInt32 ? 1 : 0;
    });
}

int mlvc_backend_run(mlvc_backend* backend, const void* const* inputs, uint16_t* const* outputs)
{
    return guard([&] {
        const auto ins = shapes(backend, false);
        const auto types = hip(backend).io_dtypes(false);
        std::vector<mlvc::Tensor> ts;
        for (std::size_t i = 0; i < ins.size(); ++i) {
            mlvc::Tensor t;
            t.shape = ins[i];
            std::size_t n = 1;
            for (auto d : t.shape) n *= static_cast<std::size_t>(d);
            if (types[i] == mlvc::TensorDataType::kInt32) {
                const auto* p = static_cast<const std::int32_t*>(inputs[i]);
                t.data = std::vector<std::int32_t>(p, p + n);
            } else {
                const auto* p = static_cast<const mlvc::Float16Storage*>(inputs[i]);
                t.data = std::vector<mlvc::Float16Storage>(p, p + n);
            }
            ts.push_back(std::move(t));
        }
        const auto outs = backend->impl->run(ts);
        for (std::size_t i = 0; i < outs.size(); ++i) std::memcpy(outputs[i], outs[i].raw_data(), outs[i].byte_size());
    });
}

int mlvc_backend_reset_state(mlvc_backend* backend)
{
    return guard([&] { backend->impl->reset_state(); });
}

int mlvc_backend_available(char* buf, size_t len)
{
    return guard([&] {
        std::string s;
        for (const auto& n : mlvc::available_backends()) s += (s.empty() ? "" : ",") + n;
        copy_str(s, buf, len);
    });
}

int mlvc_hip_backend_upload_inputs(mlvc_backend* backend, const void* const* inputs)
{
    return guard([&] {
        const std::size_t n = shapes(backend, false).size();
        hip(backend).upload_inputs(std::vector<const void*>(inputs, inputs + n));
    });
}

// ---- BufferedCodecBackend ----------------------------------------------

int mlvc_backend_configure_codec_io(mlvc_backend* backend, int width, int height, int model_width, int model_height,
                                    float pixel_range, int pad_left, int pad_right, int pad_top, int pad_bottom,
                                    int rotated, size_t slots)
{
    return guard([&] {
        mlvc::CodecIoConfig c;
        c.width = width;
        c.height = height;
        c.model_width = model_width;
        c.model_height = model_height;
        c.pixel_range = pixel_range;
        c.padding = mlvc::FramePadding{pad_left, pad_right, pad_top, pad_bottom, rotated != 0};
        c.slots = slots;
        buffered(backend).configure_codec_io(c);
    });
}

int mlvc_backend_codec_slot_count(mlvc_backend* backend, size_t* count)
{
    return guard([&] { *count = buffered(backend).codec_slot_count(); });
}

int mlvc_backend_encoder_input_yuv(mlvc_backend* backend, size_t slot, uint8_t** y, uint8_t** u, uint8_t** v)
{
    return guard([&] {
        const auto f = buffered(backend).encoder_input_yuv(slot);
        *y = f.y().data();
        *u = f.u().data();
        *v = f.v().data();
    });
}

int mlvc_backend_submit_encoder(mlvc_backend* backend, size_t slot, int shifted_q)
{
    return guard([&] { buffered(backend).submit_encoder(slot, shifted_q); });
}

int mlvc_backend_encoder_output(mlvc_backend* backend, size_t slot, int index, const void** data, size_t* bytes)
{
    return guard([&] {
        const auto v = buffered(backend).encoder_outputs(slot).at(static_cast<std::size_t>(index));
        *data = v.raw_data();
        *bytes = v.byte_size();
    });
}

int mlvc_backend_decoder_input(mlvc_backend* backend, size_t slot, int index, void** data, size_t* bytes)
{
    return guard([&] {
        const auto v = buffered(backend).decoder_inputs(slot).at(static_cast<std::size_t>(index));
        *data = v.raw_data();
        *bytes = v.byte_size();
    });
}

int mlvc_backend_codec_tensor_count(mlvc_backend* backend, size_t slot, int is_decoder, int* count)
{
    return guard([&] {
        auto& b = buffered(backend);
        *count = static_cast<int>(is_decoder ? b.decoder_inputs(slot).size() : b.encoder_outputs(slot).size());
    });
}

int mlvc_backend_submit_decoder(mlvc_backend* backend, size_t slot, int shifted_q)
{
    return guard([&] { buffered(backend).submit_decoder(slot, shifted_q); });
}

int mlvc_backend_decoder_output_yuv(mlvc_backend* backend, size_t slot, const uint8_t** y, const uint8_t** u,
                                    const uint8_t** v)
{
    return guard([&] {
        const auto f = buffered(backend).decoder_output_yuv(slot);
        *y = f.y().data();
        *u = f.u().data();
        *v = f.v().data();
    });
}

int mlvc_backend_wait_codec_slot(mlvc_backend* backend, size_t slot)
{
    return guard([&] { buffered(backend).wait_codec_slot(slot); });
}

int mlvc_frame_padding(int width, int height, int model_width, int model_height, int* pad5)
{
    return guard([&] {
        const auto p = mlvc::frame_padding(width, height, model_width, model_height);
        pad5[0] = p.left;
        pad5[1] = p.right;
        pad5[2] = p.top;
        pad5[3] = p.bottom;
        pad5[4] = p.rotated ? 1 : 0;
    });
}

int mlvc_hip_backend_time_frames(mlvc_backend* backend, int frames, float* ms)
{
    return guard([&] { *ms = hip(backend).time_frames(frames); });
}

int mlvc_hip_backend_time_frames_each(mlvc_backend* backend, int frames, size_t flush_bytes, float* ms_each)
{
    return guard([&] {
        if (!ms_each) throw std::runtime_error("time_frames_each: null output");
        hip(backend).time_frames_each(frames, flush_bytes, ms_each);
    });
}

int mlvc_hip_backend_download_outputs(mlvc_backend* backend, uint16_t* const* outputs)
{
    return guard([&] {
        const std::size_t n = shapes(backend, true).size();
        hip(backend).download_outputs(std::vector<std::uint16_t*>(outputs, outputs + n));
    });
}

int mlvc_hip_backend_launch_count(mlvc_backend* backend, int* count)
{
    return guard([&] { *count = static_cast<int>(hip(backend).launch_count()); });
}

int mlvc_hip_backend_launch_info(mlvc_backend* backend, int index, char* name, size_t name_len, char* kind, size_t kind_len,
                                 double* flops, double* bytes)
{
    return guard([&] {
        const auto info = hip(backend).launch_info(static_cast<std::size_t>(index));
        copy_str(info.name, name, name_len);
        copy_str(info.kind, kind, kind_len);
        *flops = info.flops;
        *bytes = info.bytes;
    });
}

int mlvc_hip_backend_time_launch(mlvc_backend* backend, int index, int reps, float* ms_per_launch)
{
    return guard([&] { *ms_per_launch = hip(backend).time_launch(static_cast<std::size_t>(index), reps); });
}

int mlvc_hip_backend_time_launch_cold(mlvc_backend* backend, int index, int reps, size_t flush_bytes, float* ms_each)
{
    return guard([&] {
        if (!ms_each) throw std::runtime_error("time_launch_cold: null output");
        hip(backend).time_launch_cold(static_cast<std::size_t>(index), reps, flush_bytes, ms_each);
    });
}

int mlvc_aot_inspect(const char* model_dir, const char* model_name, int* nodes, int* tensors, uint64_t* arena_bytes,
                     uint64_t* weights_bytes)
{
    return guard([&] {
        const auto g = mlvc::aot::load_aot_graph(std::filesystem::path(model_dir), model_name);
        *nodes = static_cast<int>(g.descriptor.nodes.size());
        *tensors = static_cast<int>(g.descriptor.tensors.size()) - 1;
        *arena_bytes = g.descriptor.arena_bytes;
        *weights_bytes = g.descriptor.weights_bytes;
    });
}

int mlvc_model_config_json(const char* model_dir, char* buf, size_t len)
{
    return guard([&] {
        const mlvc::ModelConfig c = mlvc::load_model_config(std::filesystem::path(model_dir));
        auto list = [](const std::vector<int>& v) {
            std::string s = "[";
            for (std::size_t i = 0; i < v.size(); ++i) s += (i ? "," : "") + std::to_string(v[i]);
            return s + "]";
        };
        auto opt = [](const std::optional<int>& v) { return v ? std::to_string(*v) : std::string("null"); };
        char range[64];
        std::snprintf(range, sizeof(range), "%.9g", static_cast<double>(c.pixel_range));
        std::string j = "{";
        j += "\"name\":\"" + c.name + "\",\"model_version\":\"" + c.model_version + "\"";
        j += ",\"model_width\":" + std::to_string(c.model_width) + ",\"model_height\":" + std::to_string(c.model_height);
        j += ",\"pixel_range\":" + std::string(range);
        j += ",\"qp_num\":" + std::to_string(c.qp_num) + ",\"total_qp_num\":" + std::to_string(c.total_qp_num);
        j += ",\"frame_index_map\":" + list(c.frame_index_map) + ",\"qp_shift\":" + list(c.qp_shift);
        j += ",\"feature_channels\":" + std::to_string(c.feature_channels) + ",\"latent_channels\":" +
             std::to_string(c.latent_channels) + ",\"hyperprior_channels\":" + std::to_string(c.hyperprior_channels);
        j += ",\"downsample_feature\":" + std::to_string(c.downsample_feature) + ",\"downsample_latent\":" +
             std::to_string(c.downsample_latent) + ",\"downsample_hyperprior\":" + std::to_string(c.downsample_hyperprior);
        j += ",\"y_scale_repeat\":" + std::to_string(c.y_scale_repeat) + ",\"iframe_period\":" + opt(c.iframe_period) +
             ",\"reset_period\":" + opt(c.reset_period) + ",\"disable_feature_reset\":" +
             (c.disable_feature_reset ? "true" : "false");
        j += ",\"feature_hw\":[" + std::to_string(c.feature_height()) + "," + std::to_string(c.feature_width()) + "]";
        j += ",\"latent_hw\":[" + std::to_string(c.latent_height()) + "," + std::to_string(c.latent_width()) + "]";
        j += ",\"hyperprior_hw\":[" + std::to_string(c.hyperprior_height()) + "," + std::to_string(c.hyperprior_width()) + "]";
        j += "}";
        if (j.size() + 1 > len) throw std::runtime_error("buffer too small for the model configuration");
        copy_str(j, buf, len);
    });
}


int mlvc_model_verify_bundle(const char* model_dir)
{
    return guard([&] { mlvc::verify_model_bundle(*mlvc::make_model_asset_reader(std::filesystem::path(model_dir))); });
}

int mlvc_model_bundle_json(const char* model_dir, char* buf, size_t len)
{
    return guard([&] {
        const auto assets = mlvc::make_model_asset_reader(std::filesystem::path(model_dir));
        const auto b = mlvc::wire::parse_model_file(assets->read_binary("model_bundle.pb"), "model_bundle.pb",
                                                    mlvc::wire::parse_bundle);
        auto quoted = [](const std::string& v) {
            std::string q = "\"";
            for (char c : v) {
                if (c == '"' || c == '\\') q += '\\';
                if (static_cast<unsigned char>(c) < 0x20) throw std::runtime_error("model bundle string holds a control character");
                q += c;
            }
            return q + "\"";
        };
        std::string j = "{\"profile\":" + quoted(b.profile) + ",\"model_version\":" + quoted(b.model_version) +
                        ",\"width\":" + std::to_string(b.width) + ",\"height\":" + std::to_string(b.height) + ",\"artifacts\":[";
        for (std::size_t i = 0; i < b.artifacts.size(); ++i)
            j += (i ? "," : "") + std::string("{\"path\":") + quoted(b.artifacts[i].path) +
                 ",\"size\":" + std::to_string(b.artifacts[i].size_bytes) + "}";
        j += "]}";
        if (j.size() + 1 > len) throw std::runtime_error("buffer too small for the model bundle description");
        copy_str(j, buf, len);
    });
}

int mlvc_model_embedded_profiles(char* buf, size_t len)
{
    return guard([&] {
        std::string s;
        for (const auto& p : mlvc::list_embedded_model_profiles()) s += (s.empty() ? "" : "\n") + p;
        if (s.size() + 1 > len) throw std::runtime_error("buffer too small for the embedded profile list");
        copy_str(s, buf, len);
    });
}

int mlvc_model_default_location(char* buf, size_t len)
{
    return guard([&] {
        const std::string s = mlvc::default_model_location().generic_string();
        if (s.size() + 1 > len) throw std::runtime_error("buffer too small for the default model location");
        copy_str(s, buf, len);
    });
}

int mlvc_synth_configs(char* buf, size_t len)
{
    return guard([&] {
        std::string s;
        for (const auto& n : mlvc::synth::synthetic_configs()) s += (s.empty() ? "" : ",") + n;
        copy_str(s, buf, len);
    });
}

int mlvc_synth_write(const char* config, const char* out_dir, uint64_t seed)
{
    return guard([&] {
        mlvc::synth::SyntheticModel info;
        const auto g = mlvc::synth::build_synthetic(config, seed, &info);
        g.write_directory(out_dir, info.model_name, info.profile);
    });
}

int mlvc_synth_input(const char* config, int index, int frame, uint64_t seed, uint16_t* dst, size_t count)
{
    return guard([&] {
        const auto v = mlvc::synth::synthetic_input(config, static_cast<std::size_t>(index), frame, seed);
        if (v.size() != count) throw std::runtime_error("synthetic input size mismatch");
        std::memcpy(dst, v.data(), count * 2);
    });
}

int mlvc_synth_bindings(const char* config, int64_t* pairs, int max_pairs, int* n_pairs, int* frames)
{
    return guard([&] {
        const auto info = mlvc::synth::synthetic_info(config);
        *n_pairs = static_cast<int>(info.state_bindings.size());
        *frames = info.frames;
        for (int i = 0; i < *n_pairs && i < max_pairs; ++i) {
            pairs[2 * i] = static_cast<int64_t>(info.state_bindings[static_cast<std::size_t>(i)].input_index);
            pairs[2 * i + 1] = static_cast<int64_t>(info.state_bindings[static_cast<std::size_t>(i)].output_index);
        }
    });
}

}  // extern "C"
