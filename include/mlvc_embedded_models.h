/* Embedded model image: model bundles compiled into a binary, read through
 * "embedded:<profile>" locations.
 *
 * Replaces the reference's linked model section (core/src/model_assets.cpp:
 * 12-83: mlvc_embedded_models_start/_end around an .incbin of the packed
 * bundles, and an index of (profile, path, offset, size) compiled in from a
 * generated mlvc_embedded_models_index.inc; packed by tools/python/
 * mlvc_tools/package.py:247-306 with every asset 16-byte aligned).
 *
 * Here the runtime references the four symbols below weakly. An image object
 * (written by mlvc.cpp_amd/python/mlvc_embed.py: an assembly file that
 * .incbin's the packed data between the start and end labels, and a C file
 * with the index) defines them, either linked into libmlvc_hip.so (build.py
 * with MLVC_EMBED_MODEL_ROOT set) or in a shared library loaded with global
 * symbol scope before it. With none defined, the build behaves like the
 * reference built without embedded models. */
#ifndef MLVC_EMBEDDED_MODELS_H
#define MLVC_EMBEDDED_MODELS_H

#ifdef __cplusplus
extern "C" {
#endif

/* One packed asset: bytes [offset, offset + size) of the data between
 * mlvc_embedded_models_start and mlvc_embedded_models_end are the file
 * `path` (generic relative path, e.g. "aot/MLVCEncoder/graph.pb") of the
 * bundle `profile` (one path component). */
struct mlvc_embedded_model_asset {
    const char* profile;
    const char* path;
    unsigned long long offset;
    unsigned long long size;
};

extern const unsigned char mlvc_embedded_models_start[];
extern const unsigned char mlvc_embedded_models_end[];
extern const struct mlvc_embedded_model_asset mlvc_embedded_models_index[];
extern const unsigned long long mlvc_embedded_models_count;

#ifdef __cplusplus
}
#endif
#endif
