"""Schema-3 graph format: wire codec, loader validation, arena plans, SHA.

* The C++ writer's graph.pb / metadata.pb are decoded with the protobuf
  library's own parser (descriptors built here from the reference schema
  proto/mlvc_model.proto:30-107), and files encoded by the protobuf library
  (packed and unpacked repeated fields, fields out of order, unknown fields)
  are accepted by the C++ loader.
* Rejections mirror decode_graph (runtime/src/aot_graph.cpp:110-284) and the
  reference's tests/unit/model_proto_tests.cpp:59-123: every require() of
  decode_graph is reached by at least one case (REJECTIONS), with the
  reference's message, plus the parse and checkpoint/weights-size checks.
* Arena non-overlap of live tensors (reference tests/unit/aot_tests.py:99-106)
  for every synthetic workload, and weights_sha256 == hashlib.sha256.
"""

import hashlib

import numpy as np
import pytest
from google.protobuf import descriptor_pb2 as dpb
from google.protobuf import descriptor_pool, message_factory

import graphs
import mlvc_hip

F = dpb.FieldDescriptorProto


def _schema():
    fdp = dpb.FileDescriptorProto(name="mlvc_model_test.proto", package="mlvc.wire", syntax="proto3")

    def msg(name, fields, oneofs=()):
        m = fdp.message_type.add(name=name)
        for o in oneofs:
            m.oneof_decl.add(name=o)
        for f in fields:
            name_, num, typ, rep = f[:4]
            fd = m.field.add(name=name_, number=num, type=typ,
                             label=F.LABEL_REPEATED if rep else F.LABEL_OPTIONAL)
            if len(f) > 4 and f[4]:
                fd.type_name = f[4]
            if len(f) > 5:
                fd.oneof_index = f[5]
        return m

    u32, u64, i64, s32, flt, byt, st, mt, en, bl = (F.TYPE_UINT32, F.TYPE_UINT64, F.TYPE_INT64, F.TYPE_SINT32, F.TYPE_FLOAT,
                                                   F.TYPE_BYTES, F.TYPE_STRING, F.TYPE_MESSAGE, F.TYPE_ENUM, F.TYPE_BOOL)
    e = fdp.enum_type.add(name="DataType")
    for i, n in enumerate(["DATA_TYPE_UNSPECIFIED", "FP16", "INT32", "INT64"]):
        e.value.add(name=n, number=i)
    e = fdp.enum_type.add(name="OpKind")
    for n, i in [("OP_UNSPECIFIED", 0)] + list(graphs.OPS.items()):
        e.value.add(name=n, number=i)
    msg("ConvAttributes", [("strides", 1, u32, 1), ("pads", 2, u32, 1), ("dilations", 3, u32, 1), ("groups", 4, u32, 0)])
    msg("AxisAttributes", [("axis", 1, s32, 0)])
    msg("ActivationAttributes", [("alpha", 1, flt, 0)])
    msg("PixelAttributes", [("block_size", 1, u32, 0)])
    msg("Node", [("op", 1, en, 0, ".mlvc.wire.OpKind"), ("inputs", 2, u32, 1), ("outputs", 3, u32, 1),
                 ("conv", 4, mt, 0, ".mlvc.wire.ConvAttributes", 0), ("axis", 5, mt, 0, ".mlvc.wire.AxisAttributes", 0),
                 ("activation", 6, mt, 0, ".mlvc.wire.ActivationAttributes", 0),
                 ("pixel", 7, mt, 0, ".mlvc.wire.PixelAttributes", 0)], ["attributes"])
    msg("ArenaAllocation", [("offset", 1, u64, 0), ("size_bytes", 2, u64, 0), ("birth", 3, u32, 0), ("death", 4, u32, 0)])
    msg("WeightLocation", [("offset", 1, u64, 0), ("size_bytes", 2, u64, 0)])
    msg("TensorDescriptor", [("id", 1, u32, 0), ("name", 2, st, 0), ("dtype", 3, en, 0, ".mlvc.wire.DataType"),
                             ("shape", 4, i64, 1), ("arena", 5, mt, 0, ".mlvc.wire.ArenaAllocation", 0),
                             ("weight", 6, mt, 0, ".mlvc.wire.WeightLocation", 0)], ["storage"])
    msg("Graph", [("schema_version", 1, u32, 0), ("checkpoint_sha256", 2, byt, 0),
                  ("tensors", 3, mt, 1, ".mlvc.wire.TensorDescriptor"), ("inputs", 4, u32, 1), ("outputs", 5, u32, 1),
                  ("nodes", 6, mt, 1, ".mlvc.wire.Node"), ("arena_bytes", 7, u64, 0), ("arena_alignment", 8, u32, 0),
                  ("weights_bytes", 9, u64, 0), ("weights_sha256", 10, byt, 0)])
    msg("ModelMetadata", [("schema_version", 1, u32, 0), ("profile", 2, st, 0), ("model_version", 3, st, 0),
                          ("checkpoint_sha256", 4, byt, 0), ("width", 5, u32, 0), ("height", 6, u32, 0),
                          ("pixel_range", 7, flt, 0)])
    pool = descriptor_pool.DescriptorPool()
    pool.Add(fdp)
    get = lambda n: message_factory.GetMessageClass(pool.FindMessageTypeByName("mlvc.wire." + n))  # noqa: E731
    return get("Graph"), get("ModelMetadata")


Graph, Meta = _schema()


def _load_pb(d, model):
    g = Graph()
    g.ParseFromString((d / "aot" / model / "graph.pb").read_bytes())
    m = Meta()
    m.ParseFromString((d / "metadata.pb").read_bytes())
    return g, m


@pytest.mark.parametrize("config", ["conv3x3_184x320", "conv_sweep_640x368", "dwblock_tiny", "mlvc_s_tiny",
                                    "mlvc_1920x1088"])
def test_cpp_writer_against_protobuf_and_arena_invariant(tmp_path, config):
    mlvc_hip.synth_write(config, tmp_path, 0)
    g, m = _load_pb(tmp_path, config)
    info = mlvc_hip.aot_inspect(tmp_path, config)
    assert g.schema_version == 3 and g.arena_alignment == 256
    assert len(g.nodes) == info["nodes"] and len(g.tensors) == info["tensors"]
    assert g.checkpoint_sha256 == m.checkpoint_sha256 and len(g.checkpoint_sha256) == 32
    weights = (tmp_path / "aot" / config / "weights.bin").read_bytes()
    assert g.weights_bytes == len(weights) == info["weights_bytes"]
    assert g.weights_sha256 == hashlib.sha256(weights).digest()
    # Arena: live intervals [birth, death] that overlap never share bytes.
    slots = [(t.arena.offset, t.arena.size_bytes, t.arena.birth, t.arena.death) for t in g.tensors if t.HasField("arena")]
    for t in g.tensors:
        if t.HasField("weight"):
            assert t.weight.offset % 256 == 0
        if t.HasField("arena"):
            assert t.arena.offset % 256 == 0 and t.arena.offset + t.arena.size_bytes <= g.arena_bytes
    for i, (o1, s1, b1, d1) in enumerate(slots):
        for o2, s2, b2, d2 in slots[i + 1:]:
            if b1 <= d2 and b2 <= d1:
                assert o1 + s1 <= o2 or o2 + s2 <= o1, "live tensors overlap in the arena"
    for i, n in enumerate(g.nodes):
        (out,) = n.outputs
        assert g.tensors[out - 1].arena.birth == i


def _protobuf_graph(unpacked: bool):
    g = Graph(schema_version=3, checkpoint_sha256=b"c" * 32, weights_sha256=b"w" * 32, arena_alignment=256,
              arena_bytes=4096, weights_bytes=512)
    g.tensors.add(id=1, name="x", dtype=1, shape=[1, 4, 2, 2])
    g.tensors.add(id=2, name="w", dtype=1, shape=[4, 4, 1, 1]).weight.CopyFrom(
        g.tensors[0].weight.__class__(offset=0, size_bytes=32))
    g.tensors.add(id=3, name="y", dtype=1, shape=[1, 4, 2, 2]).arena.CopyFrom(
        g.tensors[0].arena.__class__(offset=0, size_bytes=256, birth=0, death=1))
    g.inputs.append(1)
    g.outputs.append(3)
    n = g.nodes.add(op=6, inputs=[1, 2, 0], outputs=[3])
    n.conv.strides.extend([1, 1])
    n.conv.pads.extend([0, 0, 0, 0])
    n.conv.dilations.extend([1, 1])
    n.conv.groups = 1
    data = g.SerializeToString()
    if unpacked:
        # Re-encode every packed field one element per tag, fields reversed.
        data = _unpack_all(data)
    return data


def _fields(buf):
    i, out = 0, []
    while i < len(buf):
        key, i = _varint(buf, i)
        f, wt = key >> 3, key & 7
        if wt == 0:
            v, i = _varint(buf, i)
            out.append((f, wt, v))
        elif wt == 2:
            ln, i = _varint(buf, i)
            out.append((f, wt, buf[i:i + ln]))
            i += ln
        elif wt == 5:
            out.append((f, wt, buf[i:i + 4]))
            i += 4
        else:
            raise ValueError(wt)
    return out


def _varint(buf, i):
    v, s = 0, 0
    while True:
        b = buf[i]
        i += 1
        v |= (b & 0x7F) << s
        s += 7
        if not b & 0x80:
            return v, i


PACKED = {"graph": {4, 5}, "tensor": {4}, "node": {2, 3}, "conv": {1, 2, 3}}


def _reencode(buf, kind):
    out = b""
    for f, wt, v in reversed(_fields(buf)):
        if wt == 2 and f in PACKED.get(kind, ()):
            j = 0
            while j < len(v):
                x, j = _varint(v, j)
                out += graphs.tag(f, 0) + graphs.varint(x)
        elif wt == 2 and (kind, f) in {("graph", 3), ("graph", 6), ("node", 4)}:
            sub = {("graph", 3): "tensor", ("graph", 6): "node", ("node", 4): "conv"}[(kind, f)]
            out += graphs.f_bytes(f, _reencode(v, sub), always=True)
        elif wt == 2:
            out += graphs.f_bytes(f, bytes(v), always=True)
        elif wt == 0:
            out += graphs.tag(f, 0) + graphs.varint(v)
        else:
            out += graphs.tag(f, wt) + bytes(v)
    # An unknown field must be skipped.
    out += graphs.tag(99, 2) + graphs.varint(3) + b"abc"
    return out


def _unpack_all(data):
    return _reencode(data, "graph")


def _write_raw(d, graph_pb, checkpoint=b"c" * 32, weights=512):
    (d / "aot" / "m").mkdir(parents=True, exist_ok=True)
    (d / "aot" / "m" / "graph.pb").write_bytes(graph_pb)
    (d / "aot" / "m" / "weights.bin").write_bytes(b"\0" * weights)
    (d / "metadata.pb").write_bytes(Meta(schema_version=1, checkpoint_sha256=checkpoint).SerializeToString())


@pytest.mark.parametrize("unpacked", [False, True])
def test_loader_accepts_protobuf_encodings(tmp_path, unpacked):
    _write_raw(tmp_path, _protobuf_graph(unpacked))
    info = mlvc_hip.aot_inspect(tmp_path, "m")
    assert info["nodes"] == 1 and info["tensors"] == 3 and info["arena_bytes"] == 4096


def _conv_graph(**kw):
    g = graphs.Graph()
    x = g.input("x", [1, 4, 4, 4])
    w = g.weight_fp16("w", np.zeros((4, 4, 3, 3)))
    y = g.conv("y", x, w, 0, (1, 1), (1, 1, 1, 1))
    g.output(y)
    for k, v in kw.items():
        setattr(g, k, v)
    return g


def _expect_reject(tmp_path, g, message):
    g.write(tmp_path, "m")
    with pytest.raises(mlvc_hip.MlvcError, match=message):
        mlvc_hip.aot_inspect(tmp_path, "m")


def test_reject_bad_schema(tmp_path):
    _expect_reject(tmp_path, _conv_graph(schema=2), "unsupported schema")


def test_reject_missing_sha(tmp_path):
    _expect_reject(tmp_path, _conv_graph(checkpoint=b"short"), "SHA-256 provenance")


def test_reject_arena_alignment(tmp_path):
    _expect_reject(tmp_path, _conv_graph(arena_alignment=64), "arena configuration")


def test_reject_duplicate_id(tmp_path):
    g = _conv_graph()
    g.tensors[1]["id"] = 1
    _expect_reject(tmp_path, g, "duplicate tensor ID or name|tensor ID range")


def test_reject_forward_reference(tmp_path):
    g = graphs.Graph()
    x = g.input("x", [1, 4, 4, 4])
    a = g.leaky_relu("a", x)
    b = g.leaky_relu("b", a)
    g.nodes[0]["inputs"] = [b]  # node 0 reads node 1's output
    g.output(b)
    _expect_reject(tmp_path, g, "unresolved operand")


def test_reject_misaligned_weight(tmp_path):
    g = _conv_graph()
    st = g.tensors[1]["storage"]
    g.tensors[1]["storage"] = ("weight", st[1] + 2, st[2])
    g.weights.extend(b"\0" * 8)
    _expect_reject(tmp_path, g, "weight extent")


def test_reject_asymmetric_pads_and_dilation(tmp_path):
    g = _conv_graph()
    g.nodes[0]["attr"] = ("conv", [1, 1], [1, 1, 0, 0], [1, 1], 1)
    _expect_reject(tmp_path, g, "asymmetric")
    g = _conv_graph()
    g.nodes[0]["attr"] = ("conv", [1, 1], [1, 1, 1, 1], [2, 2], 1)
    _expect_reject(tmp_path / "d", g, "dilation")


def test_reject_wrong_attributes(tmp_path):
    g = _conv_graph()
    g.nodes[0]["attr"] = ("pixel", 2)
    _expect_reject(tmp_path, g, "convolution contract")
    g = graphs.Graph()
    x = g.input("x", [1, 4, 4, 4])
    y = g.leaky_relu("y", x, float("nan"))
    g.output(y)
    _expect_reject(tmp_path / "nan", g, "activation contract")


def test_reject_birth_and_checkpoint_mismatch(tmp_path):
    g = _conv_graph()
    g.tensors[2]["storage"][3] = 1  # born at node 1, produced by node 0
    _expect_reject(tmp_path, g, "tensor birth|arena extent")
    g = _conv_graph()
    g.write(tmp_path / "ck", "m")
    (tmp_path / "ck" / "metadata.pb").write_bytes(Meta(schema_version=1, checkpoint_sha256=b"z" * 32).SerializeToString())
    with pytest.raises(mlvc_hip.MlvcError, match="checkpoint differs"):
        mlvc_hip.aot_inspect(tmp_path / "ck", "m")


def test_reject_weights_size(tmp_path):
    g = _conv_graph()
    g.write(tmp_path, "m")
    (tmp_path / "aot" / "m" / "weights.bin").write_bytes(b"\0" * 100)
    with pytest.raises(mlvc_hip.MlvcError, match="weights size"):
        mlvc_hip.aot_inspect(tmp_path, "m")


def test_synthetic_generator_is_deterministic(tmp_path):
    for sub in ("a", "b"):
        mlvc_hip.synth_write("mlvc_s_tiny", tmp_path / sub, 0)
    for f in ("aot/mlvc_s_tiny/graph.pb", "aot/mlvc_s_tiny/weights.bin", "metadata.pb"):
        assert (tmp_path / "a" / f).read_bytes() == (tmp_path / "b" / f).read_bytes()
    mlvc_hip.synth_write("mlvc_s_tiny", tmp_path / "c", 1)
    assert (tmp_path / "a" / "aot/mlvc_s_tiny/weights.bin").read_bytes() != \
           (tmp_path / "c" / "aot/mlvc_s_tiny/weights.bin").read_bytes()
    x0 = mlvc_hip.synth_input("mlvc_s_tiny", 0, 0, (1, 3, 32, 64))
    x1 = mlvc_hip.synth_input("mlvc_s_tiny", 0, 1, (1, 3, 32, 64))
    f = graphs.to_float(x0)
    assert not (x0 == x1).all() and f.min() >= 0.0 and f.max() <= 1.0


# ---- every decode_graph rejection (runtime/src/aot_graph.cpp:110-284) ---------------------------

def _one_input(shape=(1, 4, 4, 4), dtype=graphs.FP16):
    g = graphs.Graph()
    x = g.input("x", list(shape), dtype)
    return g, x


def _unary_graph(op="SIGMOID", extra_inputs=(), attr=None):
    g, x = _one_input()
    y = g.node(op, [x, *extra_inputs], "y", g.shape(x), attr)
    g.output(y)
    return g


def _case_weights_sha():
    g = _conv_graph()
    g.weights_sha = b"x" * 5
    return g


def _case_no_tensors():
    return graphs.Graph()


def _case_no_nodes():
    g, x = _one_input()
    g.output(x)
    return g


def _case_rank():
    g, x = _one_input((1, 2, 2, 2, 2))
    g.output(g.leaky_relu("y", x))
    return g


def _case_zero_dim():
    g, x = _one_input((1, 0, 4, 4))
    g.output(g.leaky_relu("y", x))
    return g


def _case_dtype(dtype):
    def make():
        g, x = _one_input(dtype=dtype)
        y = g.leaky_relu("y", x)
        g.output(y)
        return g
    return make


def _case_input_with_arena():
    g, x = _one_input()
    y = g.leaky_relu("y", x)
    g.inputs.append(y)
    g.output(y)
    return g


def _case_input_twice():
    g, x = _one_input()
    g.inputs.append(x)
    g.output(g.leaky_relu("y", x))
    return g


def _case_concat_without_axis():
    g, x = _one_input()
    y = g.node("CONCAT", [x, x], "y", [1, 8, 4, 4])
    g.output(y)
    return g


def _case_gather_three_inputs():
    g, x = _one_input()
    i = g.weight("i", np.zeros(1, np.int64), graphs.INT64)
    y = g.node("GATHER", [x, i, i], "y", [1, 1, 4, 4], ("axis", 1))
    g.output(y)
    return g


def _case_binary_with_attr():
    g, x = _one_input()
    y = g.node("ADD", [x, x], "y", g.shape(x), ("axis", 1))
    g.output(y)
    return g


def _case_binary_absent_operand():
    g, x = _one_input()
    y = g.node("MUL", [x, 0], "y", g.shape(x))
    g.output(y)
    return g


def _case_conv_absent_weight():
    g, x = _one_input()
    y = g.node("CONV", [x, 0, 0], "y", g.shape(x), ("conv", [1, 1], [0, 0, 0, 0], [1, 1], 1))
    g.output(y)
    return g


def _case_clip_four_inputs():
    g, x = _one_input()
    y = g.node("CLIP", [x, 0, 0, 0], "y", g.shape(x))
    g.output(y)
    return g


def _case_slice_two_inputs():
    g, x = _one_input()
    s = g.weight("s", np.zeros(1, np.int64), graphs.INT64)
    y = g.node("SLICE", [x, s], "y", g.shape(x))
    g.output(y)
    return g


def _case_slice_absent_ends():
    g, x = _one_input()
    s = g.weight("s", np.zeros(1, np.int64), graphs.INT64)
    y = g.node("SLICE", [x, s, 0], "y", g.shape(x))
    g.output(y)
    return g


def _case_pixel_block(block):
    def make():
        g, x = _one_input((1, 16, 4, 4))
        y = g.node("DEPTH_TO_SPACE", [x], "y", [1, 4, 8, 8], None if block is None else ("pixel", block))
        g.output(y)
        return g
    return make


def _case_conv_attr(strides, pads, dil, groups):
    def make():
        g = _conv_graph()
        g.nodes[0]["attr"] = ("conv", strides, pads, dil, groups)
        return g
    return make


def _case_op(op):
    def make():
        g = _unary_graph()
        g.nodes[0]["op"] = op
        return g
    return make


def _case_two_outputs():
    g = _unary_graph()
    g.nodes[0]["outputs"].append(1)
    return g


def _case_output_is_weight():
    g, x = _one_input()
    w = g.weight_fp16("w", np.zeros((1, 4, 4, 4)))
    g.nodes.append(dict(op=graphs.OPS["LEAKY_RELU"], inputs=[x], outputs=[w], attr=("activation", 0.1)))
    g.output(w)
    return g


def _case_output_written_twice():
    g, x = _one_input()
    y = g.leaky_relu("y", x)
    g.nodes.append(dict(op=graphs.OPS["LEAKY_RELU"], inputs=[x], outputs=[y], attr=("activation", 0.1)))
    g.output(y)
    return g


def _case_graph_output_twice():
    g = _unary_graph()
    g.output(g.outputs[0])
    return g


def _case_graph_output_unknown():
    g = _unary_graph()
    g.outputs.append(77)
    return g


def _case_arena_misaligned():
    g = _unary_graph()
    g.tensors[1]["storage"][1] = 8
    return g


def _case_arena_death_past_end():
    g = _unary_graph()
    g.tensors[1]["storage"][4] = 5
    return g


def _case_int32_weight():
    g = _conv_graph()
    st = g.tensors[1]["storage"]
    g.tensors[1]["dtype"] = graphs.INT32
    g.tensors[1]["shape"] = [4, 4, 3, 3]
    g.tensors[1]["storage"] = ("weight", st[1], 4 * 4 * 9 * 4)
    g.weights.extend(b"\0" * (4 * 4 * 9 * 2))
    return g


def _case_empty_name():
    g = _unary_graph()
    g.tensors[0]["name"] = ""
    return g


def _case_duplicate_name():
    g = _unary_graph()
    g.tensors[1]["name"] = "x"
    return g


def _case_id_out_of_range():
    g = _unary_graph()
    g.tensors[1]["id"] = 9
    return g


REJECTIONS = [
    ("weights_sha", _case_weights_sha, "missing SHA-256 provenance"),
    ("no_tensors", _case_no_tensors, "tensor count"),
    ("no_nodes", _case_no_nodes, "empty graph"),
    ("rank5", _case_rank, "tensor rank"),
    ("zero_dim", _case_zero_dim, "tensor extent overflow"),
    ("dtype_unspecified", _case_dtype(0), "unsupported dtype"),
    ("dtype_unknown", _case_dtype(7), "unsupported dtype"),
    ("int64_activation", _case_dtype(graphs.INT64), "runtime int64 tensor"),
    ("input_with_arena", _case_input_with_arena, "input ID or storage"),
    ("input_twice", _case_input_twice, "input ID or storage"),
    ("concat_no_axis", _case_concat_without_axis, "axis contract"),
    ("gather_3_inputs", _case_gather_three_inputs, "axis contract"),
    ("binary_attr", _case_binary_with_attr, "binary contract"),
    ("binary_absent", _case_binary_absent_operand, "absent required operand"),
    ("conv_absent_w", _case_conv_absent_weight, "absent required operand"),
    ("clip_4_inputs", _case_clip_four_inputs, "clip contract"),
    ("slice_2_inputs", _case_slice_two_inputs, "slice contract"),
    ("slice_absent_ends", _case_slice_absent_ends, "absent required operand"),
    ("unary_2_inputs", lambda: _unary_graph("ROUND", extra_inputs=(1,)), "unary contract"),
    ("unary_attr", lambda: _unary_graph("RECIPROCAL", attr=("axis", 0)), "unary contract"),
    ("pixel_no_attr", _case_pixel_block(None), "pixel layout contract"),
    ("pixel_block0", _case_pixel_block(0), "invalid positive attribute"),
    ("conv_groups0", _case_conv_attr([1, 1], [1, 1, 1, 1], [1, 1], 0), "invalid positive attribute"),
    ("conv_3_strides", _case_conv_attr([1, 1, 1], [1, 1, 1, 1], [1, 1], 1), "attribute dimension count"),
    ("conv_3_pads", _case_conv_attr([1, 1], [1, 1, 1], [1, 1], 1), "attribute dimension count"),
    ("conv_stride0", _case_conv_attr([0, 1], [1, 1, 1, 1], [1, 1], 1), "invalid attribute dimension"),
    ("conv_dil0", _case_conv_attr([1, 1], [1, 1, 1, 1], [0, 1], 1), "invalid attribute dimension"),
    ("conv_pad_huge", _case_conv_attr([1, 1], [1 << 31, 1, 1 << 31, 1], [1, 1], 1), "invalid attribute dimension"),
    ("op_unspecified", _case_op(0), "unknown operator"),
    ("op_unknown", _case_op(42), "unknown operator"),
    ("two_outputs", _case_two_outputs, "output ID"),
    ("output_is_weight", _case_output_is_weight, "duplicate output or missing arena"),
    ("output_written_twice", _case_output_written_twice, "duplicate output or missing arena"),
    ("graph_output_twice", _case_graph_output_twice, "graph output"),
    ("graph_output_unknown", _case_graph_output_unknown, "graph output"),
    ("arena_misaligned", _case_arena_misaligned, "arena extent"),
    ("arena_death", _case_arena_death_past_end, "arena extent"),
    ("int32_weight", _case_int32_weight, "weight extent"),
    ("empty_name", _case_empty_name, "duplicate tensor ID or name"),
    ("duplicate_name", _case_duplicate_name, "duplicate tensor ID or name"),
    ("id_out_of_range", _case_id_out_of_range, "tensor ID range"),
]


@pytest.mark.parametrize("make,message", [c[1:] for c in REJECTIONS], ids=[c[0] for c in REJECTIONS])
def test_every_decode_rejection(tmp_path, make, message):
    g = make()
    g.write(tmp_path, "m")
    with pytest.raises(mlvc_hip.MlvcError) as e:
        mlvc_hip.aot_inspect(tmp_path, "m")
    # require() prefixes its condition (aot_graph.cpp:12-18).
    assert str(e.value).endswith("invalid AOT Protobuf graph: " + message), str(e.value)


def test_reject_unparseable_files(tmp_path):
    """parse_proto_bytes (aot_graph.cpp:95-106), labelled with the graph path (:296-298)."""
    _conv_graph().write(tmp_path, "m")
    (tmp_path / "aot" / "m" / "graph.pb").write_bytes(b"")
    with pytest.raises(mlvc_hip.MlvcError, match="invalid Protobuf model message size: aot/m/graph.pb"):
        mlvc_hip.aot_inspect(tmp_path, "m")
    (tmp_path / "aot" / "m" / "graph.pb").write_bytes(b"\x0a\xff\x01abc")  # length past the end
    with pytest.raises(mlvc_hip.MlvcError, match="invalid Protobuf model message: aot/m/graph.pb"):
        mlvc_hip.aot_inspect(tmp_path, "m")
