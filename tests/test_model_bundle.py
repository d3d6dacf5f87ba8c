"""Bundle / asset path: ModelConfig from metadata.pb checked against model_bundle.pb.

Mirrors the reference's expectations:
  - core/src/model.cpp:34-48 (validate_bundle_manifest), :50-91 (ModelConfig::validate),
    :150-183 (load_model_config);
  - tests/unit/runtime_decoupling_tests.cpp:108-160 (the synthetic 64x64 bundle) and :296-300;
  - tools/python/mlvc_tools/package.py:97-143 (artifact size and SHA-256 checks).

The metadata and bundle files are written here with a small protobuf encoder (field numbers of
mlvc_model.proto: ModelMetadata 1-21, ModelBundle 1-9, CodecContract 1-4, Artifact 1-3), so the
C++ reader is checked against an encoding it did not produce. CPU only: nothing here touches a GPU.
"""
from __future__ import annotations

import hashlib
import shutil
import struct
import sys
import pathlib

import pytest

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parents[1] / "mlvc.cpp_amd" / "python"))
import mlvc_hip  # noqa: E402


# ---- minimal protobuf encoder -------------------------------------------------------------

def _varint(v: int) -> bytes:
    out = bytearray()
    v &= (1 << 64) - 1
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(field: int, wt: int) -> bytes:
    return _varint((field << 3) | wt)


def _u(field: int, v: int) -> bytes:
    return _key(field, 0) + _varint(v)


def _bytes(field: int, v: bytes | str) -> bytes:
    if isinstance(v, str):
        v = v.encode()
    return _key(field, 2) + _varint(len(v)) + v


def _f32(field: int, v: float) -> bytes:
    return _key(field, 5) + struct.pack("<f", v)


def _f64(field: int, v: float) -> bytes:
    return _key(field, 1) + struct.pack("<d", v)


def _packed(field: int, values, enc) -> bytes:
    body = b"".join(_varint(enc(v)) for v in values)
    return _bytes(field, body)


def _zigzag(v: int) -> int:
    return (v << 1) ^ (v >> 31)


CKPT = b"c" * 32
ENTROPY = b"e" * 32

# The synthetic bundle of runtime_decoupling_tests.cpp:108-160.
BASE_META = dict(schema_version=1, profile="synthetic-v1", model_version="v1", checkpoint_sha256=CKPT,
                 width=64, height=64, pixel_range=1.0, qp_num=4, total_qp_num=8, frame_index_map=[0, 1],
                 qp_shift=[0, 2], feature_channels=2, latent_channels=4, hyperprior_channels=2,
                 downsample_feature=16, downsample_latent=16, downsample_hyperprior=2, y_scale_repeat=2,
                 iframe_period=2, reset_period=None, disable_feature_reset=True)
BASE_BUNDLE = dict(schema_version=2, profile="synthetic-v1", model_version="v1", width=64, height=64,
                   checkpoint_sha256=CKPT, entropy_model_sha256=ENTROPY, container="mlvc-nalu-v0",
                   entropy="canonical-pmf-v1", artifacts=())

_META_FIELDS = ["schema_version", "profile", "model_version", "checkpoint_sha256", "width", "height",
                "pixel_range", "qp_num", "total_qp_num", "frame_index_map", "qp_shift", "feature_channels",
                "latent_channels", "hyperprior_channels", "downsample_feature", "downsample_latent",
                "downsample_hyperprior", "y_scale_repeat", "iframe_period", "reset_period",
                "disable_feature_reset"]


def encode_metadata(m: dict) -> bytes:
    out = bytearray()
    for field, name in enumerate(_META_FIELDS, start=1):
        v = m.get(name)
        if v is None:
            continue
        if name in ("profile", "model_version", "checkpoint_sha256"):
            out += _bytes(field, v)
        elif name == "pixel_range":
            out += _f32(field, v)
        elif name == "frame_index_map":
            out += _packed(field, v, lambda x: x)
        elif name == "qp_shift":
            out += _packed(field, v, _zigzag)
        elif name == "disable_feature_reset":
            out += _u(field, int(v))
        else:
            out += _u(field, v)  # optional iframe/reset periods are written whenever present
    return bytes(out)


def encode_bundle(b: dict) -> bytes:
    contract = _bytes(1, b["container"]) + _bytes(2, b["entropy"]) + _u(3, 2) + _f64(4, 40.0)
    out = (_u(1, b["schema_version"]) + _bytes(2, b["profile"]) + _bytes(3, b["model_version"]) +
           _u(4, b["width"]) + _u(5, b["height"]) + _bytes(6, b["checkpoint_sha256"]) +
           _bytes(7, b["entropy_model_sha256"]) + _bytes(8, contract))
    for path, size, sha in b["artifacts"]:
        out += _bytes(9, _bytes(1, path) + _u(2, size) + _bytes(3, sha))
    return out


def write_model(d: pathlib.Path, meta: dict | None = None, bundle: dict | None = None,
                **meta_overrides) -> pathlib.Path:
    m = dict(BASE_META if meta is None else meta)
    m.update(meta_overrides)
    d.mkdir(parents=True, exist_ok=True)
    (d / "metadata.pb").write_bytes(encode_metadata(m))
    (d / "model_bundle.pb").write_bytes(encode_bundle(dict(BASE_BUNDLE if bundle is None else bundle)))
    return d


def _error(fn, *args) -> str:
    with pytest.raises(mlvc_hip.MlvcError) as e:
        fn(*args)
    return str(e.value)


# ---- loading and derived values --------------------------------------------------------------

def test_synthetic_bundle_loads(tmp_path):
    """runtime_decoupling_tests.cpp:296-300: name and width of the 64x64 synthetic bundle."""
    d = write_model(tmp_path / "m")
    c = mlvc_hip.model_config(d)
    assert c["name"] == "synthetic-v1" and c["model_width"] == 64 and c["model_height"] == 64
    assert c["model_version"] == "v1" and c["pixel_range"] == 1.0
    assert c["qp_num"] == 4 and c["total_qp_num"] == 8
    assert c["frame_index_map"] == [0, 1] and c["qp_shift"] == [0, 2]
    assert c["iframe_period"] == 2 and c["reset_period"] is None and c["disable_feature_reset"] is True
    # ceil(64/16) = 4; hyperprior ceil(64/(16*2)) = 2
    assert c["feature_hw"] == [4, 4] and c["latent_hw"] == [4, 4] and c["hyperprior_hw"] == [2, 2]


def test_derived_dimensions_round_up(tmp_path):
    """divide_up (model.cpp:16-25) rounds up: 1080 / 16 -> 68, 1080 / 64 -> 17, 1920 / 64 -> 30."""
    d = write_model(tmp_path / "m", width=1920, height=1080, downsample_feature=2, downsample_latent=16,
                    downsample_hyperprior=4)
    b = dict(BASE_BUNDLE, width=1920, height=1080)
    (d / "model_bundle.pb").write_bytes(encode_bundle(b))
    c = mlvc_hip.model_config(d)
    assert c["feature_hw"] == [540, 960] and c["latent_hw"] == [68, 120] and c["hyperprior_hw"] == [17, 30]
    d2 = write_model(tmp_path / "m2", width=1000, height=999, downsample_feature=3, downsample_latent=7,
                     downsample_hyperprior=5)
    (d2 / "model_bundle.pb").write_bytes(encode_bundle(dict(BASE_BUNDLE, width=1000, height=999)))
    c = mlvc_hip.model_config(d2)
    assert c["feature_hw"] == [333, 334] and c["latent_hw"] == [143, 143] and c["hyperprior_hw"] == [29, 29]


# ---- ModelConfig::validate --------------------------------------------------------------------

@pytest.mark.parametrize("overrides,message", [
    (dict(downsample_feature=0), "invalid fixed-shape model metadata"),
    (dict(downsample_latent=0), "invalid fixed-shape model metadata"),
    (dict(y_scale_repeat=0), "invalid fixed-shape model metadata"),
    (dict(latent_channels=5), "invalid fixed-shape model metadata"),        # odd latent
    (dict(latent_channels=6, y_scale_repeat=4), "invalid fixed-shape model metadata"),  # 6 % 4
    (dict(latent_channels=8, y_scale_repeat=2), "invalid fixed-shape model metadata"),  # 8/2 > 2
    (dict(total_qp_num=3), "invalid fixed-shape model metadata"),           # total < qp_num
    (dict(qp_num=0), "invalid fixed-shape model metadata"),
    (dict(pixel_range=0.0), "invalid fixed-shape model metadata"),
    (dict(pixel_range=float("inf")), "invalid fixed-shape model metadata"),
    (dict(frame_index_map=[]), "invalid fixed-shape model metadata"),
    (dict(qp_shift=[]), "invalid fixed-shape model metadata"),
    (dict(frame_index_map=[0, 2]), "model QP shift mapping is out of range"),
    (dict(qp_shift=[0, 9]), "model QP shift is outside the model range"),
    (dict(qp_shift=[0, -1]), "model QP shift is outside the model range"),
    (dict(iframe_period=0), "model I-frame period must be positive"),
    (dict(reset_period=0), "model reset period must be positive"),
    (dict(reset_period=32), "requires the dmc61sbr_e1d1 no-reset profile"),
    (dict(disable_feature_reset=False), "requires the dmc61sbr_e1d1 no-reset profile"),
    (dict(downsample_latent=1 << 16, downsample_hyperprior=1 << 16), "model downsample factor is too large"),
])
def test_invalid_metadata_rejected(tmp_path, overrides, message):
    d = write_model(tmp_path / "m", **overrides)
    err = _error(mlvc_hip.model_config, d)
    assert message in err
    # load_model_config appends the metadata location (model.cpp:176-181).
    assert err.endswith(str(d) + "/metadata.pb")


def test_integer_beyond_int_range_rejected(tmp_path):
    d = write_model(tmp_path / "m", feature_channels=1 << 31)
    assert "model integer exceeds runtime range" in _error(mlvc_hip.model_config, d)


# ---- validate_bundle_manifest ----------------------------------------------------------------

@pytest.mark.parametrize("meta_over,bundle_over", [
    (dict(schema_version=2), {}),
    ({}, dict(schema_version=1)),
    ({}, dict(profile="other")),
    ({}, dict(model_version="v2")),
    ({}, dict(width=32)),
    ({}, dict(height=32)),
    (dict(checkpoint_sha256=b"c" * 31), dict(checkpoint_sha256=b"c" * 31)),
    ({}, dict(entropy_model_sha256=b"e" * 16)),
    ({}, dict(checkpoint_sha256=b"d" * 32)),
    ({}, dict(container="mlvc-nalu-v1")),
    ({}, dict(entropy="other-pmf")),
])
def test_bundle_mismatch_rejected(tmp_path, meta_over, bundle_over):
    d = write_model(tmp_path / "m", meta=dict(BASE_META, **meta_over), bundle=dict(BASE_BUNDLE, **bundle_over))
    assert "model bundle does not match Protobuf metadata" in _error(mlvc_hip.model_config, d)


def test_missing_bundle_or_metadata(tmp_path):
    d = write_model(tmp_path / "m")
    (d / "model_bundle.pb").unlink()
    assert "model_bundle.pb" in _error(mlvc_hip.model_config, d)
    d = write_model(tmp_path / "n")
    (d / "metadata.pb").unlink()
    assert "metadata.pb" in _error(mlvc_hip.model_config, d)


def test_unparseable_files(tmp_path):
    """read_model_proto (core/src/model_proto.hpp:11-23): size and parse failures name the file."""
    d = write_model(tmp_path / "m")
    (d / "model_bundle.pb").write_bytes(b"")
    assert "invalid Protobuf model message size: model_bundle.pb" in _error(mlvc_hip.model_config, d)
    (d / "model_bundle.pb").write_bytes(b"\x12\x40short")
    assert "invalid Protobuf model message: model_bundle.pb" in _error(mlvc_hip.model_config, d)
    d = write_model(tmp_path / "n")
    (d / "metadata.pb").write_bytes(b"\x08")
    assert "invalid Protobuf model message: metadata.pb" in _error(mlvc_hip.model_config, d)


def test_embedded_locations(tmp_path):
    """model_assets.cpp: 'embedded:<profile>' selects the embedded reader; a library linked without a model
    image reports it with the reference's message, and a malformed profile is rejected before that."""
    assert "embedded models are disabled in this build (embedded:mlvc-psnr-v1)" in _error(
        mlvc_hip.model_config, "embedded:mlvc-psnr-v1")
    # A profile is one path component (model_assets.cpp:35-47).
    for bad in ("embedded:", "embedded:mlvc-psnr-v1/640x368", "embedded:a\\b"):
        assert "invalid embedded model profile" in _error(mlvc_hip.model_config, bad)


# ---- artifacts (size and SHA-256) ------------------------------------------------------------

def _synthetic_codec_dir(tmp_path) -> pathlib.Path:
    d = tmp_path / "codec"
    mlvc_hip.synth_write("codec_enc_tiny", d)
    mlvc_hip.synth_write("codec_dec_tiny", d)
    return d


def test_synthetic_codec_directory(tmp_path):
    """The synthetic codec directory carries metadata.pb and a model_bundle.pb that lists every
    artifact with its size and SHA-256; both graphs of the pair are listed."""
    d = _synthetic_codec_dir(tmp_path)
    c = mlvc_hip.model_config(d)
    assert c["model_version"] == "synthetic-v1" and c["feature_channels"] == 64
    assert c["frame_index_map"] == [0, 1, 2, 3] and c["qp_shift"] == [0, 8, 4, 8]
    mlvc_hip.verify_bundle(d)
    for rel in ("aot/MLVCEncoder/graph.pb", "aot/MLVCEncoder/weights.bin", "aot/MLVCDecoder/graph.pb",
                "aot/MLVCDecoder/weights.bin", "metadata.pb"):
        assert (d / rel).is_file()


def _artifacts(d: pathlib.Path):
    out = []
    for rel in ("metadata.pb", "aot/X/graph.pb", "aot/X/weights.bin"):
        data = (d / rel).read_bytes()
        out.append((rel, len(data), hashlib.sha256(data).digest()))
    return out


def _bundle_with_artifacts(tmp_path) -> pathlib.Path:
    d = write_model(tmp_path / "m")
    (d / "aot" / "X").mkdir(parents=True)
    (d / "aot" / "X" / "graph.pb").write_bytes(b"\x08\x03" * 40)
    (d / "aot" / "X" / "weights.bin").write_bytes(bytes(range(256)) * 9)
    (d / "model_bundle.pb").write_bytes(encode_bundle(dict(BASE_BUNDLE, artifacts=_artifacts(d))))
    return d


def test_verify_bundle_detects_tamper(tmp_path):
    d = _bundle_with_artifacts(tmp_path)
    mlvc_hip.verify_bundle(d)
    w = d / "aot" / "X" / "weights.bin"
    data = bytearray(w.read_bytes())
    data[1000] ^= 1
    w.write_bytes(bytes(data))
    assert "model bundle artifact hash mismatch: aot/X/weights.bin" in _error(mlvc_hip.verify_bundle, d)
    w.write_bytes(bytes(data[:-1]))
    assert "model bundle artifact size mismatch: aot/X/weights.bin" in _error(mlvc_hip.verify_bundle, d)
    (d / "aot" / "X" / "graph.pb").unlink()
    assert "model bundle artifact is missing: aot/X/graph.pb" in _error(mlvc_hip.verify_bundle, d)


def test_verify_bundle_rejects_malformed_entry(tmp_path):
    d = _bundle_with_artifacts(tmp_path)
    arts = _artifacts(d)
    arts[0] = (arts[0][0], arts[0][1], arts[0][2][:31])
    (d / "model_bundle.pb").write_bytes(encode_bundle(dict(BASE_BUNDLE, artifacts=arts)))
    assert "model bundle artifact entry is malformed" in _error(mlvc_hip.verify_bundle, d)


def test_synthetic_codec_tamper(tmp_path):
    d = _synthetic_codec_dir(tmp_path)
    shutil.copy(d / "aot" / "MLVCDecoder" / "weights.bin", tmp_path / "w")
    p = d / "aot" / "MLVCDecoder" / "weights.bin"
    data = bytearray(p.read_bytes())
    data[len(data) // 2] ^= 0x40
    p.write_bytes(bytes(data))
    assert "hash mismatch: aot/MLVCDecoder/weights.bin" in _error(mlvc_hip.verify_bundle, d)
    shutil.copy(tmp_path / "w", p)
    mlvc_hip.verify_bundle(d)
