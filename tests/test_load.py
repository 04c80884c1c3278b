"""The model-file side (include/beatlm_load.h through beatlm_amd/load.py):

* the safetensors reader against the reference's own reader tests
  (crates/beatlm/src/load/reader.rs:260-430) and, file by file, against the
  `safetensors` 0.8.0 Python package (the version of the crate the reference
  pins; a library, not the reference): the same files accepted and refused,
  the same tensors read;
* inventories and their check reports (load/inventory.rs:247-357);
* the Depth Anything V2 inventory and configuration rules
  (load/depth_anything_v2.rs:622-972: 24 785 089 parameters, shapes, roles);
* the layout conversions (model/mod.rs:452-558) and the bicubic position
  resampling (model/positions.rs:148-216), the latter also against torch's
  `interpolate(mode="bicubic", align_corners=False)`.

CPU only.
"""

import ctypes as C
import itertools
import random
import struct

import numpy as np
import pytest
import safetensors
import safetensors.numpy as stn
import torch

from beatlm_amd import ir, load


def f32_bytes(values):
    return np.asarray(values, "<f4").tobytes()


def header_file(header: str, data: bytes = b"") -> bytes:
    h = header.encode()
    return struct.pack("<Q", len(h)) + h + data


def file_of(entries):
    """A safetensors file from (name, numpy array) pairs, written by the
    safetensors package."""
    return stn.save(dict(entries))


# ---- the reader: the reference's cases ---------------------------------------------


def test_tensors_come_back_with_name_dtype_shape_and_bytes():
    weights = np.arange(1, 7, dtype="<f4").reshape(2, 3)
    ids = np.array([7, 8, 9], np.uint8)
    a = load.Archive.parse(file_of([("w", weights), ("ids", ids)]))
    assert len(a) == 2
    w = a.get("w")
    assert (w.dtype, w.shape) == (load.StoredType.F32, (2, 3))
    assert bytes(w.data) == weights.tobytes()
    assert w.element_count() == 6
    i = a.get("ids")
    assert (i.dtype, i.shape) == (load.StoredType.U8, (3,))
    assert bytes(i.data) == ids.tobytes()
    assert np.array_equal(w.numpy(), weights)


def test_iteration_is_in_name_order():
    a = load.Archive.parse(file_of([(n, np.zeros(1, np.float32)) for n in "bac"]))
    assert [n for n, _ in a] == ["a", "b", "c"]


def test_tensor_bytes_borrow_from_the_buffer():
    buf = file_of([("w", np.ones(4, np.float32))])
    a = load.Archive.parse(buf)
    t = a.get("w")
    base = C.cast(C.c_char_p(a._keep), C.c_void_p).value
    at = C.addressof(C.c_uint8.from_buffer(t.data))
    assert base <= at and at + len(t.data) <= base + len(buf)


def test_parameter_count_sums_every_element():
    a = load.Archive.parse(file_of([("a", np.zeros((2, 3), np.float32)), ("b", np.zeros(4, np.float32)),
                                    ("scalar", np.zeros((), np.float32))]))
    assert a.parameter_count() == 11


def test_a_dtype_without_a_name_is_other():
    a = load.Archive.parse(file_of([("h", np.zeros(2, np.int16))]))
    assert a.get("h").dtype == load.StoredType.OTHER


def test_a_missing_tensor_is_an_error_from_require_and_none_from_get():
    a = load.Archive.parse(file_of([("a", np.zeros(1, np.float32))]))
    assert a.get("nope") is None
    with pytest.raises(load.MissingTensor, match="nope"):
        a.require("nope")


def test_a_truncated_file_is_a_format_error():
    f = file_of([("a", np.ones(4, np.float32))])
    with pytest.raises(load.FormatError):
        load.Archive.parse(f[:-1])


def test_bytes_that_are_not_a_file_are_a_format_error():
    for bad in (b"", b"\xff" * 64):
        with pytest.raises(load.FormatError):
            load.Archive.parse(bad)


def test_an_empty_archive_is_valid():
    a = load.Archive.parse(file_of([]))
    assert a.is_empty() and a.parameter_count() == 0


def test_element_widths_are_known_for_named_types_only():
    assert load.StoredType.F32.size_bytes() == 4
    assert load.StoredType.BF16.size_bytes() == 2
    assert load.StoredType.OTHER.size_bytes() is None
    assert [str(t) for t in load.StoredType] == ["F32", "F16", "BF16", "F64", "U8", "I32", "I64", "other"]


def test_only_types_the_engine_plans_as_stored_convert():
    from beatlm_amd import hip

    assert load.StoredType.F32.to_planned() == hip.F32
    assert load.StoredType.F16.to_planned() == hip.F16
    assert load.StoredType.BF16.to_planned() is None
    assert load.StoredType.F64.to_planned() is None


def test_a_file_read_from_disk_parses_as_its_bytes_do(tmp_path):
    f = file_of([("w", np.array([[1.0, -2.0], [3.5, 0.25]], np.float32)), ("ids", np.array([7, 8, 9], np.uint8))])
    p = tmp_path / "parity.safetensors"
    p.write_bytes(f)

    def tensors(a):
        return [(n, t.dtype, t.shape, bytes(t.data)) for n, t in a]

    from_disk, from_bytes = load.Archive.open(p), load.Archive.parse(load.read_file(p))
    assert tensors(from_disk) == tensors(from_bytes) == tensors(load.Archive.parse(f))
    assert from_disk.parameter_count() == from_bytes.parameter_count()


def test_an_unreadable_path_is_an_io_error_naming_the_path():
    with pytest.raises(load.IoError, match="file.safetensors"):
        load.Archive.open("/definitely/not/a/file.safetensors")
    with pytest.raises(load.IoError, match="file.safetensors"):
        load.read_file("/definitely/not/a/file.safetensors")


# ---- the reader against safetensors 0.8.0, file by file --------------------------------

STORED = {"F32": load.StoredType.F32, "F16": load.StoredType.F16, "BF16": load.StoredType.BF16,
          "F64": load.StoredType.F64, "U8": load.StoredType.U8, "I32": load.StoredType.I32, "I64": load.StoredType.I64}


def same_verdict(data: bytes):
    """Both readers accept `data` and read the same tensors, or both refuse it."""
    try:
        want = safetensors.deserialize(data)
    except Exception:
        want = None
    try:
        got = load.Archive.parse(data)
    except load.FormatError:
        got = None
    assert (got is None) == (want is None), (data[:200], want is None)
    if want is None:
        return
    expect = sorted((n, STORED.get(d["dtype"], load.StoredType.OTHER), tuple(d["shape"]), bytes(d["data"]))
                    for n, d in want)
    assert [(n, t.dtype, t.shape, bytes(t.data)) for n, t in got] == expect


T = '"dtype":"F32","shape":[1],"data_offsets":[0,4]'
Z4 = b"\0" * 4
CORPUS = [
    header_file('{"a":{%s}}' % T, Z4),
    header_file('{"a":{%s,"x":1}}' % T, Z4),                                   # unknown field: ignored
    header_file('{"a":{%s},"a":{%s}}' % (T, T), Z4),                           # a name twice: the last
    header_file('{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},'
                '"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', b"\0" * 8),
    header_file('{"a":{%s,"dtype":"F32"}}' % T, Z4),                           # a field twice
    header_file('{"__metadata__":null,"a":{%s}}' % T, Z4),
    header_file('{"__metadata__":{"k":"v","k":"w"},"a":{%s}}' % T, Z4),
    header_file('{"__metadata__":{"k":1},"a":{%s}}' % T, Z4),
    header_file('{"__metadata__":{"k":null},"a":{%s}}' % T, Z4),
    header_file('{"__metadata__":"x","a":{%s}}' % T, Z4),
    header_file('{"__metadata__":{},"__metadata__":{},"a":{%s}}' % T, Z4),
    header_file('{"__metadata__":{"dtype":"F32"},"a":{%s}}' % T, Z4),
    header_file(' \n\t{"a":{%s}}   ' % T, Z4),
    header_file('{"a":{%s}}x' % T, Z4),
    header_file('{"a":{%s}}\0' % T, Z4),
    header_file(''), header_file('   '), header_file('{}'), header_file('[]'), header_file('{"a":null}'),
    header_file('{"a":{"dtype":"F32","shape":[],"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{"dtype":"F32","shape":[0],"data_offsets":[0,0]},"b":{%s}}' % T, Z4),
    header_file('{"a":{"dtype":"F32","shape":[1.0],"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{"dtype":"F32","shape":[1e0],"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{"dtype":"F32","shape":[-0],"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{"dtype":"F32","shape":[+1],"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{"dtype":"F32","shape":[01],"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{"dtype":"F32","shape":[1,],"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{%s},}' % T, Z4),
    header_file('{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4,4]}}', Z4),
    header_file('{"a":{"dtype":"F32","shape":[1],"data_offsets":[0]}}', Z4),
    header_file('{"a":{"dtype":"F32","shape":[1],"data_offsets":{"0":0}}}', Z4),
    header_file('{"a":{"dtype":"F32","shape":null,"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{"dtype":1,"shape":[1],"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{"dtype":"F32","shape":[1],"data_offsets":[4,8]}}', b"\0" * 8),
    header_file('{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{%s}}' % T, b"\0" * 5), header_file('{"a":{%s}}' % T, b"\0" * 3),
    header_file('{"a":{"dtype":"F32","shape":[1]}}', Z4),
    header_file('{"a":{"dtype":"F4","shape":[3],"data_offsets":[0,2]}}', b"\0" * 2),
    header_file('{"a":{"dtype":"F4","shape":[2],"data_offsets":[0,1]}}', b"\0"),
    header_file('{"a":{"dtype":"F6_E2M3","shape":[4],"data_offsets":[0,3]}}', b"\0" * 3),
    header_file('{"a\\u00e9\\n":{%s}}' % T, Z4), header_file('{"\\u00E9":{%s}}' % T, Z4),
    header_file('{"\\ud83d\\ude00":{%s}}' % T, Z4), header_file('{"\\ud83d":{%s}}' % T, Z4),
    header_file('{"\\ude00":{%s}}' % T, Z4), header_file('{"a\\x":{%s}}' % T, Z4),
    header_file('{"a\tb":{%s}}' % T, Z4), header_file('{"":{%s}}' % T, Z4),
    header_file('{"b":{"dtype":"F32","shape":[1],"data_offsets":[4,8]},"a":{%s}}' % T, b"\0" * 8),
    header_file('{"b":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},"a":{%s}}' % T, Z4),
    header_file('{"a":{"dtype":"F32","shape":[0],"data_offsets":[4,0]}}'),
    header_file('{"a":{%s,"x":[true,false,null,{"y":"z"},1.5e-3,-2]}}' % T, Z4),
    header_file('{"a":{%s,"x":tru}}' % T, Z4),
    header_file('{"a":{"dtype":"F32","shape":[18446744073709551615,2],"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{"dtype":"F32","shape":[18446744073709551616],"data_offsets":[0,4]}}', Z4),
    header_file('{ "a" : { "dtype" : "F32" , "shape" : [ 1 ] , "data_offsets" : [ 0 , 4 ] } }', Z4),
    header_file('{"a":{"dtype":"U8","shape":[1,1,1,1,1,1,1,1,1,1],"data_offsets":[0,1]}}', b"\0"),
    header_file('{"a":{"dtype":"F128","shape":[1],"data_offsets":[0,4]}}', Z4),
    header_file('{"a":{"dtype":"f32","shape":[1],"data_offsets":[0,4]}}', Z4),
    b"\x01\0\0\0", struct.pack("<Q", 100_000_001) + b"{}", struct.pack("<Q", 10) + b"{}",
    struct.pack("<Q", 9) + b'{"\xff":{}}' + b"", b"",
]
DTYPE_NAMES = ["BOOL", "F4", "F6_E2M3", "F6_E3M2", "U8", "I8", "F8_E5M2", "F8_E4M3", "F8_E8M0", "F8_E4M3FNUZ",
               "F8_E5M2FNUZ", "I16", "U16", "F16", "BF16", "I32", "U32", "F32", "C64", "F64", "I64", "U64"]


@pytest.mark.parametrize("i", range(len(CORPUS)))
def test_the_reader_agrees_with_safetensors_on_hand_made_headers(i):
    same_verdict(CORPUS[i])


@pytest.mark.parametrize("dtype", DTYPE_NAMES)
@pytest.mark.parametrize("count,nbytes", [(8, 8), (8, 16), (8, 32), (8, 64), (4, 2), (4, 3), (3, 2)])
def test_every_element_type_has_the_width_safetensors_gives_it(dtype, count, nbytes):
    same_verdict(header_file('{"t":{"dtype":"%s","shape":[%d],"data_offsets":[0,%d]}}' % (dtype, count, nbytes),
                             bytes(range(nbytes))))


def random_file(rng: random.Random) -> bytes:
    types = [np.float32, np.float16, np.float64, np.uint8, np.int8, np.int16, np.int32, np.int64, np.uint16,
             np.uint32, np.uint64, np.bool_]
    entries = {}
    for _ in range(rng.randint(0, 6)):
        name = "".join(rng.choice("abcxyz._0123é") for _ in range(rng.randint(0, 8)))
        shape = tuple(rng.randint(0, 4) for _ in range(rng.randint(0, 4)))
        t = rng.choice(types)
        entries[name] = (np.random.default_rng(rng.randint(0, 999)).integers(0, 2, shape) if t is np.bool_
                         else np.random.default_rng(rng.randint(0, 999)).integers(0, 100, shape)).astype(t)
    return stn.save(entries, metadata={"k": "v"} if rng.random() < 0.3 else None)


def test_the_reader_agrees_with_safetensors_on_random_and_mutated_files():
    rng = random.Random(7)
    for _ in range(300):
        f = random_file(rng)
        same_verdict(f)
        n = struct.unpack("<Q", f[:8])[0]
        for _ in range(4):
            b = bytearray(f)
            how = rng.randrange(5)
            if how == 0 and n:
                b[8 + rng.randrange(n)] = rng.randrange(256)            # a header byte
            elif how == 1:
                b = b[: rng.randrange(len(b) + 1)]                      # truncated
            elif how == 2:
                b += bytes(rng.randrange(1, 5))                          # longer
            elif how == 3 and n:
                i = 8 + rng.randrange(n)
                b[i:i] = rng.choice([b" ", b",", b"0", b"]", b"}", b'"', b"\\"])  # a character more
            else:
                b[:8] = struct.pack("<Q", max(0, n + rng.randint(-3, 3)))  # the length off
            same_verdict(bytes(b))


# ---- inventories ---------------------------------------------------------------------


def spec(name, shape, dtype=load.StoredType.F32, role=None):
    return load.TensorSpec(name, dtype, tuple(shape), role or load.Role(99))


def zeros(name, shape):
    return (name, np.zeros(shape, np.float32))


def small_inventory():
    return load.Inventory([spec("a", (2, 3)), spec("b", (4,))])


def test_a_file_with_exactly_the_tensors_is_exact():
    r = small_inventory().check(load.Archive.parse(file_of([zeros("a", (2, 3)), zeros("b", (4,))])))
    assert r.is_exact(), str(r)
    assert (r.expected_parameters, r.file_parameters) == (10, 10)
    assert str(r) == "the file matches the inventory exactly: 10 parameters"


def test_every_difference_is_reported_not_just_the_first():
    inv = load.Inventory([spec("gone", (1,)), spec("also_gone", (1,)), spec("reshaped", (2, 3)),
                          spec("retyped", (2,)), spec("fine", (5,))])
    f = file_of([zeros("reshaped", (3, 2)), ("retyped", np.zeros(2, np.float16)), zeros("fine", (5,)),
                 zeros("extra", (7,)), zeros("another_extra", (1,))])
    r = inv.check(load.Archive.parse(f))
    assert not r.is_exact()
    assert r.missing == ["gone", "also_gone"]
    assert r.unexpected == ["another_extra", "extra"]
    assert [m.name for m in r.mismatched] == ["reshaped", "retyped"]
    assert r.mismatched[0].expected.shape == (2, 3) and r.mismatched[0].found.shape == (3, 2)
    assert r.mismatched[1].found.dtype == load.StoredType.F16
    assert r.expected_parameters == 1 + 1 + 6 + 2 + 5
    assert r.file_parameters == 6 + 2 + 5 + 7 + 1


def test_the_rendered_report_names_every_difference():
    r = small_inventory().check(load.Archive.parse(file_of([zeros("a", (3, 2)), zeros("stray", (1,))])))
    text = str(r)
    assert text.startswith("the file does not match the inventory: 1 missing, 1 unexpected, 1 mismatched "
                           "(inventory 10 parameters, file 7)")
    assert "missing    b" in text
    assert "unexpected stray" in text
    assert "mismatch   a: expected F32 [2, 3], found F32 [3, 2]" in text


def test_a_repeated_name_is_refused():
    with pytest.raises(load.DuplicateName, match="`a`"):
        load.Inventory([spec("a", (1,)), spec("a", (2,))])


def test_specs_are_found_by_name_and_by_role():
    inv = load.Inventory([spec("x", (1,), role=load.Role(1)), spec("y", (2,), role=load.Role(2))])
    assert inv.get("y").role == load.Role(2)
    assert inv.by_role(load.Role(1)).name == "x"
    assert inv.get("z") is None and inv.by_role(load.Role(3)) is None
    assert [s.name for s in inv] == ["x", "y"] and len(inv) == 2


# ---- Depth Anything V2 -----------------------------------------------------------------


def tiny():
    return ir.DepthConfig(image_size=4, patch_size=2, hidden_size=8, num_layers=4, num_heads=2,
                          out_indices=(1, 2, 3, 4), neck_hidden_sizes=(2, 4, 6, 8), fusion_hidden_size=4,
                          head_hidden_size=2)


def zero_file(inv, skip=""):
    return file_of([(s.name, np.zeros(s.shape, np.float32)) for s in inv if s.name != skip])


def test_the_small_model_has_the_published_parameter_count():
    assert load.inventory(ir.DepthConfig.small()).parameter_count() == 24_785_089


def test_names_are_distinct_and_roles_are_distinct():
    specs = list(load.inventory(ir.DepthConfig.small()))
    assert len({s.name for s in specs}) == len(specs) == len({s.role for s in specs})


def test_the_layers_follow_the_configuration():
    inv = load.inventory(ir.DepthConfig.small())
    q = inv.get("backbone.encoder.layer.11.attention.attention.query.weight")
    assert q.shape == (384, 384)
    assert q.role == load.block_role(11, load.QUERY, load.WEIGHT)
    assert inv.get("backbone.encoder.layer.12.norm1.weight") is None
    assert inv.get("backbone.encoder.layer.0.mlp.fc1.weight").shape == (1536, 384)
    assert inv.get("backbone.embeddings.position_embeddings").shape == (1, 37 * 37 + 1, 384)
    assert inv.get("backbone.embeddings.patch_embeddings.projection.weight").shape == (384, 3, 14, 14)


def test_the_resampling_tensors_follow_the_stage():
    inv = load.inventory(ir.DepthConfig.small())

    def shape(name):
        s = inv.get(name)
        return s and s.shape

    assert shape("neck.reassemble_stage.layers.0.resize.weight") == (48, 48, 4, 4)
    assert shape("neck.reassemble_stage.layers.1.resize.weight") == (96, 96, 2, 2)
    assert shape("neck.reassemble_stage.layers.2.resize.weight") is None
    assert shape("neck.reassemble_stage.layers.2.resize.bias") is None
    assert shape("neck.reassemble_stage.layers.3.resize.weight") == (384, 384, 3, 3)


def test_the_neck_convolutions_have_no_bias_and_the_head_ends_in_one_channel():
    inv = load.inventory(ir.DepthConfig.small())
    assert inv.get("neck.convs.3.weight").shape == (64, 384, 3, 3)
    assert inv.get("neck.convs.3.bias") is None
    assert inv.get("head.conv3.weight").shape == (1, 32, 1, 1)
    assert inv.get("head.conv1.weight").shape == (32, 64, 3, 3)


def test_roles_find_the_tensor():
    inv = load.inventory(ir.DepthConfig.small())
    found = inv.by_role(load.Role(load.FUSION, 3, load.RESIDUAL, load.BIAS, unit=0, conv=1))
    assert found.name == "neck.fusion_stage.layers.3.residual_layer1.convolution2.bias"
    assert found.shape == (64,)


def test_without_a_mask_token_the_inventory_lacks_it():
    from dataclasses import replace

    inv = load.inventory(replace(ir.DepthConfig.small(), mask_token=False))
    assert inv.get("backbone.embeddings.mask_token") is None
    assert inv.parameter_count() == 24_785_089 - 384


def test_a_file_written_from_the_inventory_checks_exact():
    inv = load.inventory(tiny())
    r = inv.check(load.Archive.parse(zero_file(inv)))
    assert r.is_exact(), str(r)
    assert r.file_parameters == inv.parameter_count()


def test_a_missing_tensor_is_named():
    inv = load.inventory(tiny())
    gone = "backbone.encoder.layer.2.mlp.fc2.weight"
    r = inv.check(load.Archive.parse(zero_file(inv, gone)))
    assert r.missing == [gone] and not r.unexpected and not r.mismatched


def test_the_v5_attention_names_are_not_in_the_inventory():
    inv = load.inventory(tiny())
    assert inv.get("backbone.encoder.layer.0.attention.q_proj.weight") is None
    assert inv.get("backbone.encoder.layer.0.attention.o_proj.weight") is None


@pytest.mark.parametrize("change,variant", [
    (dict(num_heads=5), "HeadsDoNotDivideHidden"),
    (dict(image_size=520), "ImageNotWholePatches"),
    (dict(out_indices=(3, 6, 9, 13)), "OutIndexOutOfRange"),
    (dict(out_indices=(0, 6, 9, 12)), "OutIndexOutOfRange"),
    (dict(neck_hidden_sizes=(48, 96, 192)), "StageCountMismatch"),
    (dict(fusion_hidden_size=63), "FusionWidthOdd"),
    (dict(hidden_size=0), "Zero"),
    (dict(reassemble=(("up", 0), ("up", 2), ("keep",), ("down", 2))), "Zero"),
    (dict(reassemble=(("up", 4), ("up", 2), ("keep",), ("down", 1))), "ResampleByOne"),
    (dict(out_indices=(3, 9, 6, 12)), "OutIndicesNotIncreasing"),
    (dict(out_indices=(3, 6, 6, 12)), "OutIndicesNotIncreasing"),
])
def test_invalid_configurations_are_refused(change, variant):
    from dataclasses import replace

    with pytest.raises(load.ConfigError) as e:
        load.inventory(replace(ir.DepthConfig.small(), **change))
    assert e.value.variant == variant
    if variant == "OutIndexOutOfRange" and 13 in change["out_indices"]:
        assert "13" in str(e.value)
    if variant == "ResampleByOne":
        assert "stage 3" in str(e.value)
    if change.get("hidden_size") == 0:
        assert "hidden_size" in str(e.value)


# ---- conversions ---------------------------------------------------------------------


def test_a_linear_weight_is_transposed_and_a_convolution_becomes_hwio():
    t, cols = load.convert([1, 2, 3, 4, 5, 6], (2, 3), load.LINEAR)
    assert (t.tolist(), cols) == ([1, 4, 2, 5, 3, 6], 2)
    t, cols = load.convert([0, 1, 10, 11], (2, 1, 2, 1), load.CONV)
    assert (t.tolist(), cols) == ([0, 10, 1, 11], 2)
    stored = [100 * i + 10 * o + x for i in range(2) for o in range(3) for x in range(2)]
    t, cols = load.convert(stored, (2, 3, 1, 2), load.CONV_TRANSPOSE)
    hwio = [100 * i + 10 * o + x for x in range(2) for i in range(2) for o in range(3)]
    assert (t.tolist(), cols) == (hwio, 3)
    with pytest.raises(load.ModelError):
        load.convert([1.0] * 6, (2, 3), load.CONV_TRANSPOSE)
    t, cols = load.convert([1, 2], (1, 1, 2), load.AS_STORED)
    assert (t.tolist(), cols) == ([1, 2], 2)
    with pytest.raises(load.ModelError):
        load.convert([1.0] * 6, (1, 2, 3), load.LINEAR)
    with pytest.raises(load.ModelError):
        load.convert([1.0] * 6, (2, 3), load.CONV)


def test_the_conversions_are_numpy_transposes():
    rng = np.random.default_rng(3)
    w = rng.standard_normal((5, 7)).astype(np.float32)
    assert np.array_equal(load.convert(w, w.shape, load.LINEAR)[0], w.T.ravel())
    k = rng.standard_normal((6, 4, 3, 2)).astype(np.float32)  # OIHW
    assert np.array_equal(load.convert(k, k.shape, load.CONV)[0], k.transpose(2, 3, 1, 0).ravel())
    kt = rng.standard_normal((4, 6, 2, 3)).astype(np.float32)  # [in][out][kh][kw]
    assert np.array_equal(load.convert(kt, kt.shape, load.CONV_TRANSPOSE)[0], kt.transpose(2, 3, 0, 1).ravel())


POS = [9.0, -9.0, 1.0, 10.0, 2.0, 20.0, 3.0, 30.0, 4.0, 40.0]


def test_a_position_embedding_is_resampled_behind_its_class_row():
    t, cols = load.convert(POS, (1, 5, 2), load.INTERPOLATE_POSITIONS, 1, 1)
    assert cols == 2 and t[:2].tolist() == [9.0, -9.0]
    assert abs(t[2] - 2.5) < 1e-6 and abs(t[3] - 25.0) < 1e-5
    same, _ = load.convert(POS, (1, 5, 2), load.INTERPOLATE_POSITIONS, 2, 2)
    assert same.tolist() == POS
    assert len(load.convert(POS, (1, 5, 2), load.INTERPOLATE_POSITIONS, 3, 3)[0]) == 20
    for shape, vals in (((5, 2), POS), ((1, 4, 2), [0.0] * 8)):
        with pytest.raises(load.ModelError):
            load.convert(vals, shape, load.INTERPOLATE_POSITIONS, 1, 1)


def grid_positions(grid: np.ndarray) -> tuple:
    """[g][g][c] as a stored embedding [1][1 + g g][c] with a class row of 7s."""
    g, _, c = grid.shape
    return np.concatenate([np.full(c, 7.0, np.float32), grid.astype(np.float32).ravel()]), (1, 1 + g * g, c)


def resampled(grid, h, w):
    vals, shape = grid_positions(grid)
    out, _ = load.convert(vals, shape, load.INTERPOLATE_POSITIONS, h, w)
    assert np.array_equal(out[: grid.shape[2]], np.full(grid.shape[2], 7.0, np.float32))
    return out[grid.shape[2]:].reshape(h, w, grid.shape[2])


def test_the_weights_are_keys_cubic_with_a_of_minus_three_quarters():
    # positions.rs:148-172. Halving 4 samples: output 0 reads indices
    # [0, 0, 1, 2] with weights [-0.09375, 0.59375, 0.59375, -0.09375]; a
    # one-hot column shows its weight, rows constant (their weights sum to 1
    # exactly: dyadic).
    def column(j, n=4):
        g = np.zeros((n, n, 1), np.float32)
        g[:, j, 0] = 1.0
        return g

    halved = [resampled(column(j), 2, 2)[:, 0, 0] for j in range(4)]
    assert [float(h[0]) for h in halved] == [-0.09375 + 0.59375, 0.59375, -0.09375, 0.0]
    # Output 1 reads [1, 2, 3, 3]: the sample after clamped to 3.
    assert [float(resampled(column(j), 2, 2)[0, 1, 0]) for j in range(4)] == [0.0, -0.09375, 0.59375,
                                                                                0.59375 - 0.09375]
    # Doubling 2 samples: output 0 reads position -0.25, indices [0, 0, 0, 1]
    # at t = 0.75; every weight set sums to one.
    d0 = [float(resampled(column(j, 2), 4, 4)[0, 0, 0]) for j in range(2)]
    assert abs(sum(d0) - 1.0) < 1e-6
    a = -0.75
    far = lambda x: ((a * x - 5 * a) * x + 8 * a) * x - 4 * a  # noqa: E731
    assert abs(d0[1] - far(2 - 0.75)) < 1e-6


def test_the_same_size_is_the_identity_and_a_constant_stays_constant():
    g = (np.arange(18, dtype=np.float32) * 0.25 - 1.0).reshape(3, 3, 2)
    assert np.array_equal(resampled(g, 3, 3), g)
    flat = np.full((5, 5, 3), 1.5, np.float32)
    for h, w in ((2, 2), (7, 7), (3, 6)):
        out = resampled(flat, h, w)
        assert out.shape == (h, w, 3) and np.all(np.abs(out - 1.5) < 1e-5)


def test_halving_a_row_weights_its_neighbours_by_the_cubic():
    g = np.tile(np.arange(4, dtype=np.float32) % 4, (4, 1))[..., None]
    out = resampled(g, 2, 2)
    want0 = 0.59375 - 0.09375 * 2.0
    assert abs(out[0, 0, 0] - want0) < 1e-6 and abs(out[1, 0, 0] - want0) < 1e-6


@pytest.mark.parametrize("g,h,w", [(37, 19, 19), (37, 74, 74), (37, 26, 31), (5, 7, 7), (4, 2, 2), (3, 3, 6)])
def test_the_resampling_matches_torch_bicubic(g, h, w):
    grid = np.random.default_rng(g * 100 + h).standard_normal((g, g, 6)).astype(np.float32)
    def torch_bicubic(x):
        t = torch.from_numpy(x).permute(2, 0, 1)[None]
        return torch.nn.functional.interpolate(t, size=(h, w), mode="bicubic", align_corners=False)[0].permute(1, 2, 0)

    got = resampled(grid, h, w)
    exact = torch_bicubic(grid.astype(np.float64)).numpy()
    torch32 = torch_bicubic(grid).numpy()
    # Both f32 computations round the cubic weights (the reference promises no
    # bit-identity with PyTorch, positions.rs:31-36): ours is as close to the
    # float64 result as torch's own f32 kernel is, and close to that kernel.
    assert np.max(np.abs(got - exact)) <= 2 * np.max(np.abs(torch32 - exact)) + 1e-6
    assert np.max(np.abs(got - torch32)) <= 3e-5


# ---- weight numbers ------------------------------------------------------------------


def two_part_file():
    inv = load.Inventory([spec("a", (2, 2), role=load.Role(1)), spec("b", (2, 1), role=load.Role(2)),
                          spec("c", (3,), role=load.Role(3)), spec("h", (2,), role=load.Role(4))])
    f = file_of([("a", np.array([[1, 2], [3, 4]], np.float32)), ("b", np.array([[5], [6]], np.float32)),
                 ("c", np.ones(3, np.float32)), ("h", np.ones(2, np.float16))])
    return inv, load.Archive.parse(f)


def test_parts_are_laid_side_by_side_row_by_row():
    inv, a = two_part_file()
    got = load.weight_numbers(inv, a, [load.Role(1), load.Role(2)], load.AS_STORED, 6)
    assert got.tolist() == [1, 2, 5, 3, 4, 6]
    assert load.weight_numbers(inv, a, [load.Role(1)], load.AS_STORED, 4).tolist() == [1, 2, 3, 4]


def test_a_weight_whose_sources_do_not_fit_is_refused():
    inv, a = two_part_file()
    for parts, how, n, code in [([load.Role(1), load.Role(3)], load.AS_STORED, 7, load.ERR_SOURCE_SIZE),
                                ([load.Role(1)], load.AS_STORED, 5, load.ERR_SOURCE_SIZE),
                                ([load.Role(9)], load.AS_STORED, 1, load.ERR_UNKNOWN_ROLE),
                                ([load.Role(4)], load.AS_STORED, 2, load.ERR_LAYOUT),
                                ([load.Role(3)], load.LINEAR, 3, load.ERR_CONVERT)]:
        with pytest.raises(load.LoadError) as e:
            load.weight_numbers(inv, a, parts, how, n)
        assert e.value.code == code, (parts, e.value)


def test_the_depth_models_weights_come_from_the_checkpoint_converted():
    """depth_weights on a tiny configuration: every weight of the graph, the
    encoder's by role, the decoder's by name, against numpy's own transposes
    of the stored tensors."""
    cfg = tiny()
    inv = load.inventory(cfg)
    rng = np.random.default_rng(11)
    stored = {s.name: rng.standard_normal(s.shape).astype(np.float32) for s in inv}
    a = load.Archive.parse(file_of(stored.items()))
    g = ir.Graph()
    m = ir.depth_model(g, cfg, 6)  # a 3 x 3 grid from the stored 2 x 2
    w = load.depth_weights(a, cfg, m, 6)
    e, blocks = m.encoder.embed, m.encoder.blocks
    p = "backbone.encoder.layer.1."
    assert np.array_equal(w[blocks[1].qkv_w].reshape(8, 24), np.concatenate(
        [stored[p + f"attention.attention.{k}.weight"].T for k in ("query", "key", "value")], axis=1))
    assert np.array_equal(w[blocks[1].qkv_b], np.concatenate(
        [stored[p + f"attention.attention.{k}.bias"] for k in ("query", "key", "value")]))
    assert np.array_equal(w[blocks[1].fc2_w], stored[p + "mlp.fc2.weight"].T.ravel())
    assert np.array_equal(w[blocks[3].ls2], stored["backbone.encoder.layer.3.layer_scale2.lambda1"])
    assert np.array_equal(w[e.patch_w], stored["backbone.embeddings.patch_embeddings.projection.weight"]
                          .transpose(2, 3, 1, 0).ravel())
    assert w[e.pos].size == (9 + 1) * 8
    assert np.array_equal(w[e.pos][:8], stored["backbone.embeddings.position_embeddings"][0, 0])
    names = {name: tid for tid, name, _ in m.decoder_weights}
    up = stored["neck.reassemble_stage.layers.0.resize.weight"]
    assert np.array_equal(w[names["neck.reassemble_stage.layers.0.resize.weight"]], up.transpose(2, 3, 0, 1).ravel())
    down = stored["neck.reassemble_stage.layers.3.resize.weight"]
    assert np.array_equal(w[names["neck.reassemble_stage.layers.3.resize.weight"]], down.transpose(2, 3, 1, 0).ravel())
    assert np.array_equal(w[names["head.conv3.weight"]], stored["head.conv3.weight"].transpose(2, 3, 1, 0).ravel())
    every = {tid for tid, _, _ in m.decoder_weights} | {getattr(b, n) for b in blocks for n in ir.BLOCK_WEIGHTS}
    every |= {e.patch_w, e.patch_b, e.cls, e.pos, m.encoder.final_g, m.encoder.final_b}
    assert set(w) == every
    # A checkpoint that is not exactly the inventory is refused, with the report.
    del stored["head.conv1.bias"]
    with pytest.raises(load.ModelError, match="missing    head.conv1.bias"):
        load.depth_weights(load.Archive.parse(file_of(stored.items())), cfg, m, 6)
