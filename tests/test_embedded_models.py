"""Embedded model image (include/mlvc_embedded_models.h, mlvc.cpp_amd/python/mlvc_embed.py).

Reference behaviour: core/src/model_assets.cpp:12-252 (an image of packed
bundles and a (profile, path, offset, size) index; "embedded:<profile>"
locations read from it; profiles listed in index order; the default location
prefers "mlvc-psnr-v1", else the first profile; an entry outside the data
is "embedded model index is corrupt"; a missing file is "embedded model asset
not found: <profile>/<path>"), packed as tools/python/mlvc_tools/package.py:
207-306 does (16-byte aligned assets, the manifest's profile equal to the
profile name, the bundle directory named <width>x<height>).

The image is built here as a shared library of its own and loaded with
global symbol scope before libmlvc_hip.so, so each check runs in a fresh
process. No GPU.
"""

import hashlib
import json
import pathlib
import subprocess
import sys
import textwrap

import pytest

import mlvc_embed
import mlvc_hip
import test_model_bundle as tmb

REPO = pathlib.Path(__file__).resolve().parents[1]


def _root_with(tmp_path, configs):
    """Synthetic bundles below <root>/<profile>/<WxH>/; returns (root, {profile: dir})."""
    root = tmp_path / "models"
    dirs = {}
    for config in configs:
        scratch = tmp_path / ("scratch_" + config)
        mlvc_hip.synth_write(config, scratch)
        info = mlvc_hip.bundle_info(scratch)
        d = root / info["profile"] / f"{info['width']}x{info['height']}"
        d.parent.mkdir(parents=True)
        scratch.rename(d)
        dirs[info["profile"]] = d
    return root, dirs


def _in_image_process(image_so, body: str) -> dict:
    """Runs `body` (which sets `out`) in a process that loaded the image first."""
    code = textwrap.dedent(f"""
        import ctypes, json, sys
        ctypes.CDLL({str(image_so)!r}, mode=ctypes.RTLD_GLOBAL)
        sys.path[:0] = [{str(REPO / 'mlvc.cpp_amd' / 'python')!r}]
        import mlvc_hip
        def error(fn, *a):
            try:
                fn(*a)
            except mlvc_hip.MlvcError as e:
                return str(e)
            return None
        out = {{}}
    """) + textwrap.dedent(body) + "\nprint(json.dumps(out))\n"
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


@pytest.fixture(scope="module")
def image(tmp_path_factory):
    tmp = tmp_path_factory.mktemp("embed")
    root, dirs = _root_with(tmp, ["codec_enc_tiny", "mlvc_s_tiny"])
    index = mlvc_embed.pack_model_root(root, tmp / "out")
    so = mlvc_embed.shared_library(tmp / "out", tmp / "libmodels.so")
    return so, dirs, index, tmp / "out"


def test_packed_layout(image):
    so, dirs, index, out = image
    data = (out / mlvc_embed.DATA).read_bytes()
    assert [p for p, *_ in index] == sorted(p for p, *_ in index)  # profiles in name order
    for profile, path, offset, size in index:
        assert offset % 16 == 0
        assert data[offset:offset + size] == (dirs[profile] / path).read_bytes()
    names = {(p, n) for p, n, *_ in index}
    for profile, d in dirs.items():
        want = {"model_bundle.pb"} | {a["path"] for a in mlvc_hip.bundle_info(d)["artifacts"]}
        assert {n for p, n in names if p == profile} == want


def test_embedded_locations_read_the_image(image):
    so, dirs, index, _ = image
    out = _in_image_process(so, f"""
        dirs = {json.dumps({p: str(d) for p, d in dirs.items()})}
        out["profiles"] = mlvc_hip.embedded_profiles()
        out["default"] = mlvc_hip.default_model_location()
        for p, d in dirs.items():
            loc = "embedded:" + p
            mlvc_hip.verify_bundle(loc)
            out[p] = mlvc_hip.bundle_info(loc) == mlvc_hip.bundle_info(d)
        codec = dirs["synthetic-codec_128x64"]
        out["config"] = [mlvc_hip.model_config("embedded:synthetic-codec_128x64"), mlvc_hip.model_config(codec)]
        out["enc"] = [mlvc_hip.aot_inspect("embedded:synthetic-codec_128x64", "MLVCEncoder"),
                      mlvc_hip.aot_inspect(codec, "MLVCEncoder")]
        out["tiny"] = [mlvc_hip.aot_inspect("embedded:synthetic-mlvc_s_tiny", "mlvc_s_tiny"),
                       mlvc_hip.aot_inspect(dirs["synthetic-mlvc_s_tiny"], "mlvc_s_tiny")]
        out["missing"] = error(mlvc_hip.aot_inspect, "embedded:synthetic-codec_128x64", "MLVCDecoder")
        out["unknown"] = error(mlvc_hip.model_config, "embedded:mlvc-psnr-v1")
        out["bad"] = error(mlvc_hip.model_config, "embedded:a/b")
    """)
    assert out["profiles"] == sorted(dirs)
    assert out["default"] == "embedded:" + sorted(dirs)[0]  # no mlvc-psnr-v1: the first profile
    for p in dirs:
        assert out[p] is True, p
    assert out["config"][0] == out["config"][1] and out["config"][0]["model_width"] == 128
    assert out["enc"][0] == out["enc"][1] and out["tiny"][0] == out["tiny"][1]
    assert out["missing"] == "embedded model asset not found: synthetic-codec_128x64/aot/MLVCDecoder/graph.pb"
    assert out["unknown"].startswith("embedded model asset not found: mlvc-psnr-v1/")
    assert "invalid embedded model profile" in out["bad"]


def test_default_location_prefers_mlvc_psnr_v1(tmp_path):
    root = tmp_path / "models"
    for profile in ("a-first", "mlvc-psnr-v1"):
        meta = dict(tmb.BASE_META, profile=profile)
        m = tmb.encode_metadata(meta)
        bundle = dict(tmb.BASE_BUNDLE, profile=profile,
                      artifacts=(("metadata.pb", len(m), hashlib.sha256(m).digest()),))
        tmb.write_model(root / profile / "64x64", meta=meta, bundle=bundle)
    mlvc_embed.pack_model_root(root, tmp_path / "out")
    so = mlvc_embed.shared_library(tmp_path / "out", tmp_path / "libm.so")
    out = _in_image_process(so, """
        out["profiles"] = mlvc_hip.embedded_profiles()
        out["default"] = mlvc_hip.default_model_location()
        out["name"] = mlvc_hip.model_config("embedded:mlvc-psnr-v1")["name"]
    """)
    assert out["profiles"] == ["a-first", "mlvc-psnr-v1"]
    assert out["default"] == "embedded:mlvc-psnr-v1"
    assert out["name"] == "mlvc-psnr-v1"  # that bundle's configuration, read from the image


def test_index_outside_the_data_is_corrupt(image, tmp_path):
    _, _, index, out = image
    src = (out / mlvc_embed.INDEX).read_text()
    last = index[-1]
    bad = src.replace(f"{last[2]}ULL, {last[3]}ULL", f"{last[2]}ULL, {last[3] + 1}ULL")
    assert bad != src
    d = tmp_path / "bad"
    d.mkdir()
    for name in (mlvc_embed.DATA, mlvc_embed.ASM):
        (d / name).write_bytes((out / name).read_bytes())
    (d / mlvc_embed.ASM).write_text((out / mlvc_embed.ASM).read_text().replace(str((out / mlvc_embed.DATA).resolve()),
                                                                                str((d / mlvc_embed.DATA).resolve())))
    (d / mlvc_embed.INDEX).write_text(bad)
    so = mlvc_embed.shared_library(d, tmp_path / "libbad.so")
    res = _in_image_process(so, f"""
        out["err"] = error(mlvc_hip.verify_bundle, "embedded:{last[0]}")
    """)
    assert res["err"] == "embedded model index is corrupt"


def test_packer_checks(tmp_path):
    _, dirs = _root_with(tmp_path, ["codec_enc_tiny"])
    (profile, d), = dirs.items()
    with pytest.raises(ValueError, match="bundle profile mismatch"):
        mlvc_embed.pack({"other-profile": d}, tmp_path / "o1")
    with pytest.raises(ValueError, match="invalid embedded model profile"):
        mlvc_embed.pack({"a/b": d}, tmp_path / "o2")
    wrong = d.parent / "1x1"
    d.rename(wrong)
    with pytest.raises(ValueError, match="does not match manifest dimensions"):
        mlvc_embed.pack_model_root(tmp_path / "models", tmp_path / "o3")
    (wrong / "metadata.pb").write_bytes(b"\x08\x01")
    with pytest.raises(mlvc_hip.MlvcError, match="model bundle artifact"):
        mlvc_embed.pack({profile: wrong}, tmp_path / "o4")


@pytest.mark.gpu
def test_backend_loads_from_the_image(image):
    """The "hip" backend loads a graph from "embedded:<profile>" and gives the
    same bits as from the bundle's directory (recurrent state over two frames)."""
    so, dirs, _, _ = image
    d = dirs["synthetic-mlvc_s_tiny"]
    out = _in_image_process(so, f"""
        import numpy as np
        bindings, _ = mlvc_hip.synth_bindings("mlvc_s_tiny")
        res = []
        for loc in ("embedded:synthetic-mlvc_s_tiny", {str(d)!r}):
            b = mlvc_hip.Backend(loc, "hip")
            b.load("mlvc_s_tiny", bindings)
            b.reset_state()
            frames = [b.run([mlvc_hip.synth_input("mlvc_s_tiny", 0, f, b.in_shapes[0])])[0] for f in range(2)]
            res.append(np.stack(frames))
            b.close()
        out["same"] = bool((res[0] == res[1]).all())
        out["shape"] = list(res[0].shape)
    """)
    assert out["same"], out


def test_profile_registry_selects_orders_and_checks_versions(tmp_path):
    """With a profile registry (the reference's models/profiles/profiles.json
    shape), exactly the registered profiles are embedded, in registry order,
    each manifest's model_version checked (package.py:249-271)."""
    root, dirs = _root_with(tmp_path, ["codec_enc_tiny", "mlvc_s_tiny", "dwblock_tiny"])
    names = sorted(dirs)
    versions = {p: mlvc_hip.bundle_info(d)["model_version"] for p, d in dirs.items()}
    chosen = [names[2], names[0]]  # reverse of name order; names[1] left out
    reg = tmp_path / "profiles.json"
    reg.write_text(json.dumps({"schema_version": 1, "profiles": {p: {"model_version": versions[p]} for p in chosen}}))
    index = mlvc_embed.pack_model_root(root, tmp_path / "out", reg)
    order = list(dict.fromkeys(p for p, *_ in index))
    assert order == chosen
    # Without a registry every profile directory is embedded, sorted by name.
    assert list(dict.fromkeys(p for p, *_ in mlvc_embed.pack_model_root(root, tmp_path / "all"))) == names
    bad = {"profiles": {chosen[0]: {"model_version": versions[chosen[0]] + "-other"}}}
    reg.write_text(json.dumps(bad))
    with pytest.raises(ValueError, match=f"bundle model version mismatch for {chosen[0]}"):
        mlvc_embed.pack_model_root(root, tmp_path / "out2", reg)
    # A registered profile without a bundle below the root.
    reg.write_text(json.dumps({"profiles": {"missing-profile": {"model_version": "v"}}}))
    with pytest.raises(FileNotFoundError, match="missing-profile"):
        mlvc_embed.pack_model_root(root, tmp_path / "out3", reg)
