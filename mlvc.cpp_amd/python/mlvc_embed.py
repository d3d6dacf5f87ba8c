"""Packs model bundles into an embedded model image (include/mlvc_embedded_models.h).

Replaces the reference's `package.py embed` step (tools/python/mlvc_tools/
package.py:207-306) for this library. For every profile, the bundle directory
is checked first (every artifact of model_bundle.pb present with its size
and SHA-256, through the runtime's own check; the manifest's profile equal to
the profile name; with a model root, the directory named
<width>x<height> after the manifest), then model_bundle.pb and the
artifacts it lists are appended to one payload, each at a 16-byte aligned
offset, and indexed as (profile, path, offset, size).

Outputs, in --out-dir:
  mlvc_embedded_models.bin   the payload
  mlvc_embedded_models.S     .incbin of the payload between the
                             mlvc_embedded_models_start / _end labels
  mlvc_embedded_models_index.c   the index and its length
and, with --shared PATH, a shared library of those two objects, which a
process loads with global symbol scope before libmlvc_hip.so (or build.py
links the two objects into libmlvc_hip.so itself when
MLVC_EMBED_MODEL_ROOT is set).

  python mlvc_embed.py --model-root ROOT [--profiles profiles.json] --out-dir DIR [--shared libmodels.so]
  python mlvc_embed.py --bundle PROFILE=DIR [--bundle ...] --out-dir DIR
"""

from __future__ import annotations

import argparse
import json
import pathlib
import subprocess
import sys

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent))

import mlvc_hip  # noqa: E402

REPO = pathlib.Path(__file__).resolve().parents[2]
ALIGN = 16
DATA, ASM, INDEX = "mlvc_embedded_models.bin", "mlvc_embedded_models.S", "mlvc_embedded_models_index.c"


def check_profile(profile: str) -> None:
    """A profile is one path component (model_assets.cpp:35-47) of printable ASCII."""
    if not profile or "/" in profile or "\\" in profile:
        raise ValueError(f"invalid embedded model profile: {profile}")
    _c_string(profile)


def _c_string(s: str) -> str:
    if not s.isascii() or not s.isprintable():
        raise ValueError(f"embedded model names must be printable ASCII: {s!r}")
    return json.dumps(s)  # for printable ASCII, JSON string escapes are C escapes


def find_bundle(model_root: pathlib.Path, profile: str) -> pathlib.Path:
    """The one <model_root>/<profile>/<WxH>/ directory holding a model_bundle.pb (package.py:207-215)."""
    found = sorted((model_root / profile).glob("*/model_bundle.pb"))
    if len(found) != 1:
        raise FileNotFoundError(f"expected exactly one bundle for {profile} below {model_root / profile}, "
                                f"found {len(found)}")
    return found[0].parent


def pack(bundles: dict[str, pathlib.Path], out_dir: pathlib.Path, check_dir_name: bool = False,
         model_versions: dict[str, str] | None = None) -> list[tuple]:
    """Writes the payload, assembly and index files for `bundles` (profile -> bundle directory, in index
    order) into out_dir and returns the index entries (profile, path, offset, size). With
    model_versions (profile -> registered model_version), each manifest's model_version must equal
    its profile's."""
    out_dir = pathlib.Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    payload = bytearray()
    index = []
    for profile, d in bundles.items():
        check_profile(profile)
        d = pathlib.Path(d)
        mlvc_hip.verify_bundle(d)
        info = mlvc_hip.bundle_info(d)
        if info["profile"] != profile:
            raise ValueError(f"bundle profile mismatch: {d} describes {info['profile']!r}, expected {profile!r}")
        if model_versions is not None and info["model_version"] != model_versions[profile]:
            raise ValueError(f"bundle model version mismatch for {profile}")
        if check_dir_name and d.name != f"{info['width']}x{info['height']}":
            raise ValueError(f"model bundle directory {d.name!r} does not match manifest dimensions "
                             f"'{info['width']}x{info['height']}'")
        for name in ["model_bundle.pb"] + [a["path"] for a in info["artifacts"]]:
            _c_string(name)
            payload.extend(b"\0" * (-len(payload) % ALIGN))
            content = (d / name).read_bytes()
            index.append((profile, name, len(payload), len(content)))
            payload.extend(content)
    data = out_dir / DATA
    data.write_bytes(bytes(payload))
    if '"' in str(data.resolve()) or "\\" in str(data.resolve()):
        raise ValueError(f"output path not usable in .incbin: {data}")
    (out_dir / ASM).write_text(
        '.section .rodata.mlvc_embedded_models,"a",%progbits\n'
        ".balign 16\n"
        ".globl mlvc_embedded_models_start\n"
        ".type mlvc_embedded_models_start, %object\n"
        "mlvc_embedded_models_start:\n"
        f'.incbin "{data.resolve()}"\n'
        ".globl mlvc_embedded_models_end\n"
        ".type mlvc_embedded_models_end, %object\n"
        "mlvc_embedded_models_end:\n"
        ".size mlvc_embedded_models_start, mlvc_embedded_models_end - mlvc_embedded_models_start\n"
        '.section .note.GNU-stack,"",%progbits\n')
    rows = "".join(f"    {{{_c_string(p)}, {_c_string(n)}, {o}ULL, {s}ULL}},\n" for p, n, o, s in index)
    (out_dir / INDEX).write_text(
        "/* Generated by mlvc_embed.py: index of mlvc_embedded_models.bin. */\n"
        '#include "mlvc_embedded_models.h"\n\n'
        f"const struct mlvc_embedded_model_asset mlvc_embedded_models_index[] = {{\n{rows or '    {0, 0, 0ULL, 0ULL},' + chr(10)}}};\n"
        f"const unsigned long long mlvc_embedded_models_count = {len(index)}ULL;\n")
    return index


def objects(out_dir: pathlib.Path) -> list[pathlib.Path]:
    """Compiles the image's assembly and index into position-independent objects."""
    out_dir = pathlib.Path(out_dir)
    objs = []
    for src in (ASM, INDEX):
        obj = out_dir / (src + ".o")
        subprocess.run(["gcc", "-c", "-fPIC", f"-I{REPO / 'include'}", str(out_dir / src), "-o", str(obj)], check=True)
        objs.append(obj)
    return objs


def shared_library(out_dir: pathlib.Path, so_path: pathlib.Path) -> pathlib.Path:
    """A shared library holding only the image (load it with RTLD_GLOBAL before libmlvc_hip.so)."""
    subprocess.run(["gcc", "-shared", *map(str, objects(out_dir)), "-o", str(so_path)], check=True)
    return pathlib.Path(so_path)


def load_registry(path: pathlib.Path) -> dict[str, str]:
    """Profile registry in the shape of the reference's models/profiles/profiles.json
    ({"profiles": {name: {"model_version": ...}, ...}}): profile -> model_version, in file order."""
    profiles = json.loads(pathlib.Path(path).read_text())["profiles"]
    return {name: reg["model_version"] for name, reg in profiles.items()}


def pack_model_root(model_root: pathlib.Path, out_dir: pathlib.Path, registry: pathlib.Path | None = None) -> list[tuple]:
    """Bundles below model_root, each profile directory holding exactly one <WxH>/ bundle. With a
    profile registry (package.py:249-271): exactly the registered profiles, in registry order, each
    manifest's model_version checked against its registration; other directories are not embedded.
    Without one: every profile directory, sorted by name."""
    model_root = pathlib.Path(model_root)
    versions = load_registry(registry) if registry is not None else None
    profiles = list(versions) if versions is not None else sorted(p.name for p in model_root.iterdir() if p.is_dir())
    if not profiles:
        raise FileNotFoundError(f"no model profiles below {model_root}")
    return pack({p: find_bundle(model_root, p) for p in profiles}, out_dir, check_dir_name=True,
                model_versions=versions)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--model-root", type=pathlib.Path)
    ap.add_argument("--profiles", type=pathlib.Path,
                    help="profile registry (profiles.json shape) selecting and ordering the profiles under --model-root")
    ap.add_argument("--bundle", action="append", default=[], metavar="PROFILE=DIR")
    ap.add_argument("--out-dir", type=pathlib.Path, required=True)
    ap.add_argument("--shared", type=pathlib.Path)
    args = ap.parse_args(argv)
    if bool(args.model_root) == bool(args.bundle):
        ap.error("give either --model-root or --bundle")
    if args.profiles and not args.model_root:
        ap.error("--profiles selects profiles under --model-root")
    if args.model_root:
        index = pack_model_root(args.model_root, args.out_dir, args.profiles)
    else:
        bundles = {}
        for b in args.bundle:
            profile, sep, d = b.partition("=")
            if not sep:
                ap.error(f"--bundle needs PROFILE=DIR: {b}")
            bundles[profile] = pathlib.Path(d)
        index = pack(bundles, args.out_dir)
    if args.shared:
        shared_library(args.out_dir, args.shared)
    print(f"{len(index)} assets, {len({p for p, *_ in index})} profiles", file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
