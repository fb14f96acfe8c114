"""CPU tests of the bootstrap wire format (sgl_kv_bootstrap_*): the frames the
decode side sends the prefill side, as the reference builds, parses and
encodes them (crates/sglang-srt/src/pd_bootstrap.rs:150-270, 416-494,
671-749, 1209-1270, 1421-1636).

Frames are assembled here with struct.pack from the reference tests' field
values (an independent packer: little-endian u64/i32/u32 values, packed
lists as a u32 count, u32 byte lengths, then the buffers), and the parsed
values are checked against the asserts of those tests
(tests/golden/reference_goldens.json, "bootstrap_frames"). Also covered:
every MooncakeBootstrapFrameError variant and its precedence, the integer
grammar of Rust's FromStr, the encoders' bytes against the same packer, and
the decode-layout extension (round trip; ignored by a 12-part reader).
"""
import struct

import pytest

import sgl_rocm_kv as kv


def pu64(values):
    return b"".join(struct.pack("<Q", v) for v in values)


def pi32(values):
    return b"".join(struct.pack("<i", v) for v in values)


def pu32(values):
    return b"".join(struct.pack("<I", v) for v in values)


def plist(buffers):
    """pack_list_of_buffers (pd_bootstrap.rs:1255-1270): empty for no buffers."""
    if not buffers:
        return b""
    return struct.pack("<I", len(buffers)) + b"".join(struct.pack("<I", len(b)) for b in buffers) + b"".join(buffers)


def plist_u64_header(buffers):
    """The variant http_server.rs:3120-3127 writes: u64 count and lengths
    interleaved with the buffers; the reference's decoder reads a u32 count."""
    out = struct.pack("<Q", len(buffers))
    for b in buffers:
        out += struct.pack("<Q", len(b)) + b
    return out


def kv_args_frame(d, lists=plist):
    f = [b"None", d["endpoint"].encode(), d["dst_port"].encode(), d["session"].encode(),
         pu64(d["dst_kv_ptrs"]), pu64(d.get("dst_aux_ptrs", [])),
         lists([pu64(x) for x in d.get("dst_state_data_ptrs", [])]),
         d["dst_tp_rank"].encode(), d["dst_attn_tp_size"].encode(), d["dst_kv_item_len"].encode()]
    if "dst_state_item_lens" in d:
        f.append(plist([pu32(x) for x in d["dst_state_item_lens"]]))
        f.append(plist([pu32(x) for x in d["dst_state_dim_per_tensor"]]))
    return f


def transfer_frame(d, lists=plist):
    return [str(d["room"]).encode(), d["endpoint"].encode(), d["dst_port"].encode(), d["session"].encode(),
            pi32(d["dst_kv_indices"]), d["dst_aux_index"].encode(),
            lists([pi32(x) for x in d.get("dst_state_indices", [])]),
            d["required_dst_info_num"].encode(), d["decode_prefix_len"].encode()]


@pytest.fixture
def state():
    s = kv.PrefillBootstrapState()
    yield s
    s.close()


def expect_error(variant, fn, *args, name=None, **kwargs):
    with pytest.raises(kv.KvError) as ei:
        fn(*args, **kwargs)
    assert ei.value.variant == variant, ei.value
    if name is not None:
        assert ei.value.name == name, ei.value
    return ei.value


# --- the reference tests' frames -----------------------------------------------------------------

def test_kv_args_register_frame(state, goldens):
    g = goldens["bootstrap_frames"]["kv_args_register"]
    state.ingest_mooncake_bootstrap_frame(kv_args_frame(g["frame"]))
    got = state.decode_kv_args("session-a")
    for key, want in g["expect"].items():
        assert got[key] == want, key
    assert got["decode_layout"] is None
    assert state.decode_kv_args_registration_count() == 1


def test_transfer_frames_mark_room_waiting(state, goldens):
    g = goldens["bootstrap_frames"]["transfer_rooms"]
    e = g["expect"]
    state.ingest_mooncake_bootstrap_frame(transfer_frame(g["first"]))
    assert state.transfer_status(77) == e["status_after_first"]
    state.ingest_mooncake_bootstrap_frame(transfer_frame(g["second"]))
    assert state.transfer_status(77) == e["status_after_second"]
    room = state.transfer_room(77)
    assert room["required_dst_info_num"] == e["required_dst_info_num"]
    assert room["decode_prefix_len"] == e["decode_prefix_len"]   # the first non-None one is kept
    assert room["transfer_count"] == e["transfer_count"]
    a = state.transfer(77, "session-a")
    assert a["dst_kv_indices"] == e["session_a_dst_kv_indices"]
    assert a["dst_aux_index"] == e["session_a_dst_aux_index"]
    assert a["dst_state_indices"] == e["session_a_dst_state_indices"]
    assert state.transfer(77, "session-b")["endpoint"] == e["session_b_endpoint"]
    assert state.transfer_status(78) is None


def test_remote_kv_layouts_for_room(state, goldens):
    g = goldens["bootstrap_frames"]["remote_layouts"]
    state.ingest_mooncake_bootstrap_frame(kv_args_frame(g["kv_args"]))
    state.ingest_mooncake_bootstrap_frame(transfer_frame(g["transfer"]))
    got = state.remote_kv_layouts_for_room(77)
    want = g["expect"]
    assert [s for s, _ in got] == [s for s, _ in want]
    for (_, lay), (_, w) in zip(got, want):
        for key in w:
            assert lay[key] == w[key], key
        assert lay["decode_layout"] is None


def test_http_prefill_target_offsets(state, goldens):
    """The frames of the reference's HTTP PD test (u64-header empty lists,
    which its u32 decoder reads as an empty list), then the remote page
    requests of the two decode pages: 0x9000 + 4*128 and 0x9000 + 5*128."""
    g = goldens["bootstrap_frames"]["http_prefill_target_offsets"]
    ka, tr = dict(g["kv_args"]), dict(g["transfer"])
    ka["dst_kv_item_len"] = str(ka["dst_kv_item_len"])
    tr.update(endpoint="10.0.0.9", dst_port="41001")
    state.ingest_mooncake_bootstrap_frame(kv_args_frame(ka, lists=plist_u64_header))
    state.ingest_mooncake_bootstrap_frame(transfer_frame(tr, lists=plist_u64_header))
    [(session, lay)] = state.remote_kv_layouts_for_room(34)
    assert session == "session-a"
    src = g["source"]
    reqs = kv.build_remote_page_requests(src["source_base_addr"], src["page_size_bytes"], 2, 1, [0, 1],
                                         lay["dst_kv_ptrs"], lay["dst_kv_indices"], lay["dst_kv_item_len"])
    assert list(reqs["target_offset"]) == g["expect_target_offsets"]


def test_rank_register_frames(state, goldens):
    g = goldens["bootstrap_frames"]["rank_register_frames"]
    state.ingest_mooncake_bootstrap_frame(kv_args_frame(g["kv_args"]))
    state.ingest_mooncake_bootstrap_frame(transfer_frame(g["transfer"]))
    assert state.transfer_status(99) == "WaitingForInput"
    [(s, lay)] = state.remote_kv_layouts_for_room(99)
    assert s == "decode-rank-session" and lay["dst_kv_indices"] == [0, 1, 2]


def test_decode_publisher_registration(goldens):
    """What the decode publisher registers (pd_bootstrap_server.rs:399-422),
    as this build's encoder writes it and its decoder reads it back."""
    g = goldens["bootstrap_frames"]["decode_publisher_registration"]
    frame = kv.encode_kv_args_frame(endpoint=g["endpoint"], dst_port=g["dst_port"],
                                    mooncake_session_id=g["mooncake_session_id"],
                                    dst_kv_ptrs=[g["layout"]["source_base_addr"]], dst_tp_rank=0,
                                    dst_attn_tp_size=1, dst_kv_item_len=g["layout"]["page_size_bytes"])
    s = kv.PrefillBootstrapState()
    s.ingest_mooncake_bootstrap_frame(frame)
    got = s.decode_kv_args(g["mooncake_session_id"])
    assert got["endpoint"] == g["endpoint"] and got["dst_port"] == g["dst_port"]
    assert got["dst_kv_ptrs"] == g["expect"]["dst_kv_ptrs"]
    assert got["dst_kv_item_len"] == g["expect"]["dst_kv_item_len"]


# --- encoders against the packer -----------------------------------------------------------------

def test_kv_args_encoder_bytes():
    """MooncakeDecodeKvArgsRegistration::to_frame (pd_bootstrap.rs:685-706):
    14 parts, part 12 empty and part 13 "0"."""
    got = kv.encode_kv_args_frame(endpoint="10.1.2.3", dst_port=7, mooncake_session_id="s-1",
                                  dst_kv_ptrs=[1, 2 ** 63 + 5], dst_aux_ptrs=[9],
                                  dst_state_data_ptrs=[[3, 4], []], dst_tp_rank=-2, dst_attn_tp_size=4,
                                  dst_kv_item_len=4096, dst_state_item_lens=[[16]], dst_state_dim_per_tensor=[])
    want = [b"None", b"10.1.2.3", b"7", b"s-1", pu64([1, 2 ** 63 + 5]), pu64([9]),
            plist([pu64([3, 4]), b""]), b"-2", b"4", b"4096", plist([pu32([16])]), b"", b"", b"0"]
    assert got == want


def test_transfer_encoder_bytes():
    """MooncakeDecodeTransferMetadata::to_frame (pd_bootstrap.rs:720-749);
    decode_prefix_len None is written as "0"; a dummy has empty parts 4-6."""
    got = kv.encode_transfer_frame(room=2 ** 63 - 1, endpoint="e", dst_port=65535, mooncake_session_id="s",
                                   dst_kv_indices=[-1, 7], dst_aux_index=3, dst_state_indices=[[1], [2, 3]],
                                   required_dst_info_num=2, decode_prefix_len=None)
    assert got == [b"9223372036854775807", b"e", b"65535", b"s", pi32([-1, 7]), b"3",
                   plist([pi32([1]), pi32([2, 3])]), b"2", b"0"]
    dummy = kv.encode_transfer_frame(room=5, endpoint="e", dst_port=1, mooncake_session_id="s", is_dummy=True,
                                     dst_aux_index=None, decode_prefix_len=9)
    assert dummy == [b"5", b"e", b"1", b"s", b"", b"", b"", b"1", b"9"]
    e = expect_error("MissingAuxIndex", kv.encode_transfer_frame, **dict(
        room=5, endpoint="e", dst_port=1, mooncake_session_id="sess-x", dst_aux_index=None))
    assert e.message == "Mooncake transfer metadata for sess-x needs aux index"
    expect_error("DimensionTooLarge", kv.encode_transfer_frame,
                 **dict(room=5, endpoint="e", dst_port=65536, mooncake_session_id="s"), name="dst_port")


def test_encode_then_ingest_round_trip(state):
    f = kv.encode_transfer_frame(room=12, endpoint="h", dst_port=80, mooncake_session_id="a",
                                 dst_kv_indices=[5, 6], dst_aux_index=0, required_dst_info_num=1,
                                 decode_prefix_len=128)
    state.ingest_mooncake_bootstrap_frame(f)
    t = state.transfer(12, "a")
    assert (t["dst_kv_indices"], t["decode_prefix_len"], t["is_dummy"]) == ([5, 6], 128, False)
    dummy = kv.encode_transfer_frame(room=12, endpoint="h", dst_port=80, mooncake_session_id="b", is_dummy=True,
                                     required_dst_info_num=2)
    state.ingest_mooncake_bootstrap_frame(dummy)
    assert state.transfer(12, "b")["is_dummy"] and state.transfer(12, "b")["dst_aux_index"] is None
    expect_error("MissingKvArgsRegistration", state.remote_kv_layouts_for_room, 12)
    state.ingest_mooncake_bootstrap_frame(kv.encode_kv_args_frame(
        endpoint="h", dst_port=80, mooncake_session_id="a", dst_kv_ptrs=[64], dst_kv_item_len=32))
    [(s, lay)] = state.remote_kv_layouts_for_room(12)   # the dummy session is skipped
    assert s == "a" and lay["dst_kv_ptrs"] == [64] and lay["dst_kv_indices"] == [5, 6]


# --- errors ---------------------------------------------------------------------------------------

def _ok_transfer():
    return transfer_frame({"room": "7", "endpoint": "e", "dst_port": "1", "session": "s", "dst_kv_indices": [1],
                           "dst_aux_index": "0", "required_dst_info_num": "1", "decode_prefix_len": "4"})


def _ok_kv_args():
    return kv_args_frame({"endpoint": "e", "dst_port": "1", "session": "s", "dst_kv_ptrs": [1],
                          "dst_tp_rank": "0", "dst_attn_tp_size": "1", "dst_kv_item_len": "8"})


def test_frame_errors(state):
    ing = state.ingest_mooncake_bootstrap_frame
    e = expect_error("MissingField", ing, [], name="room")
    assert e.fields[:2] == (1, 0)
    e = expect_error("MissingField", ing, _ok_kv_args()[:9], name="Mooncake KVArgs registration")
    assert e.fields[:2] == (10, 9)
    assert e.message == "Mooncake KVArgs registration frame requires at least 10 fields, got 9"
    expect_error("MissingField", ing, _ok_transfer()[:7], name="Mooncake transfer metadata")
    expect_error("Utf8Field", ing, [b"\xff"], name="room")
    bad = _ok_kv_args()
    bad[1] = b"\xc0\xaf"                                   # overlong '/'
    expect_error("Utf8Field", ing, bad, name="endpoint")
    bad = _ok_kv_args()
    bad[4] = b"\x00" * 12
    e = expect_error("BinaryLength", ing, bad, name="u64 values")
    assert e.fields[:2] == (8, 12)
    bad = _ok_kv_args()
    bad[6] = b"\x01\x00"
    expect_error("PackedListHeader", ing, bad, name="u64 lists")
    bad[6] = struct.pack("<I", 2) + struct.pack("<I", 8)
    expect_error("PackedListHeader", ing, bad, name="u64 lists")
    bad[6] = struct.pack("<II", 1, 16) + b"\x00" * 8
    expect_error("PackedListLength", ing, bad, name="u64 lists")
    bad[6] = struct.pack("<II", 1, 12) + b"\x00" * 12
    expect_error("BinaryLength", ing, bad, name="u64 values")
    bad = _ok_kv_args() + [struct.pack("<II", 1, 3) + b"\x00" * 3]
    expect_error("BinaryLength", ing, bad, name="u32 values")
    t = _ok_transfer()
    t[4] = b"\x00" * 5
    expect_error("BinaryLength", ing, t, name="i32 values")
    # the indices are checked before the room (MooncakeTransferInfo::from_frame's order)
    t[0] = b"x"
    expect_error("BinaryLength", ing, t, name="i32 values")
    assert state.transfer_status(7) is None                 # errors change nothing


@pytest.mark.parametrize("index,name,value,ok", [
    (2, "dst_port", b"65535", True), (2, "dst_port", b"65536", False), (2, "dst_port", b"+80", True),
    (2, "dst_port", b"-1", False), (2, "dst_port", b"", False), (2, "dst_port", b"+", False),
    (2, "dst_port", b" 80", False), (2, "dst_port", b"8O", False),
    (5, "dst_aux_index", b"-2147483648", True), (5, "dst_aux_index", b"2147483648", False),
    (5, "dst_aux_index", b"-", False), (5, "dst_aux_index", b"+7", True),
    (0, "room", b"9223372036854775807", True), (0, "room", b"9223372036854775808", False),
    (0, "room", b"18446744073709551616", False), (7, "required_dst_info_num", b"18446744073709551615", True),
    (8, "decode_prefix_len", b"x", False),
])
def test_integer_fields(state, index, name, value, ok):
    """The grammar of Rust's integer FromStr: optional '+' (and '-' for
    signed types), ASCII digits only, no overflow."""
    t = _ok_transfer()
    t[index] = value
    if ok:
        state.ingest_mooncake_bootstrap_frame(t)
    else:
        e = expect_error("IntegerField", state.ingest_mooncake_bootstrap_frame, t, name=name)
        assert e.message == f"{name} must be an integer, got {value.decode()}"


def test_ignored_and_optional_parts(state):
    state.ingest_mooncake_bootstrap_frame([b"WATERMARK"])
    state.ingest_mooncake_bootstrap_frame([b"STAGING_RSP", b"\xff"])
    t = _ok_transfer()[:8]                                  # no decode_prefix_len part
    state.ingest_mooncake_bootstrap_frame(t)
    assert state.transfer_room(7)["decode_prefix_len"] is None
    t = _ok_transfer()
    t[8] = b""                                              # empty is None too
    t[3] = b"s2"
    t[7] = b"2"
    state.ingest_mooncake_bootstrap_frame(t)
    assert state.transfer_room(7) == {"required_dst_info_num": 2, "decode_prefix_len": None, "transfer_count": 2}
    assert state.transfer_status(7) == "WaitingForInput"
    expect_error("MissingTransferRoom", state.remote_kv_layouts_for_room, 8)
    e = expect_error("MissingKvArgsRegistration", state.remote_kv_layouts_for_room, 7)
    assert e.message == "missing Mooncake KVArgs registration for room 7 session s"


def test_session_reregistration_replaces(state):
    a = _ok_kv_args()
    state.ingest_mooncake_bootstrap_frame(a)
    a[4] = pu64([77, 78])
    state.ingest_mooncake_bootstrap_frame(a)
    assert state.decode_kv_args("s")["dst_kv_ptrs"] == [77, 78]
    assert state.decode_kv_args_registration_count() == 2


# --- the decode-layout extension -----------------------------------------------------------------

def _layout(P=64, hnd=kv.HND, pair=False):
    if pair:
        rt = kv.KvCacheRuntimeLayout("bf16", P, 61, 1, 576, 2, 61 * (1152 + 1024), 61 * (1152 + 1024) * P)
        return kv.DecodeLayout(kv.PagedKvCacheLayout.new_with_tensor_pair(rt, 4096, 1152, 1024), kv.NHD, 0)
    rt = kv.KvCacheRuntimeLayout.for_model("bf16", P, 32, 8, 128)
    return kv.DecodeLayout(kv.PagedKvCacheLayout.new(rt, 4096), hnd, 8)


@pytest.mark.parametrize("pair", [False, True])
def test_decode_layout_round_trip(state, pair):
    dl = _layout(pair=pair)
    f = kv.encode_kv_args_frame(endpoint="e", dst_port=1, mooncake_session_id="s", dst_kv_ptrs=[0x7000],
                                dst_kv_item_len=dl.layout._c.runtime.page_size_bytes, decode_layout=dl)
    assert len(f) == 15 and len(f[14]) == 112
    assert struct.unpack_from("<II", f[14]) == (0x4C564B53, 1)
    state.ingest_mooncake_bootstrap_frame(f)
    got = state.decode_kv_args("s")["decode_layout"]
    assert got is not None and got.head_layout == dl.head_layout and got.heads == dl.heads
    for name in ("page_count", "total_byte_len", "slot_count", "bytes_per_layer_page", "tensor_pair"):
        assert getattr(got.layout._c, name) == getattr(dl.layout._c, name), name
    assert list(got.layout._c.token_bytes) == list(dl.layout._c.token_bytes)
    # A reader of the reference's 12 parts never sees it.
    s2 = kv.PrefillBootstrapState()
    s2.ingest_mooncake_bootstrap_frame(f[:12])
    assert s2.decode_kv_args("s")["decode_layout"] is None


def test_decode_layout_errors(state):
    f = kv.encode_kv_args_frame(endpoint="e", dst_port=1, mooncake_session_id="s", dst_kv_ptrs=[1],
                                decode_layout=_layout())
    for part, what in ((f[14][:100], "length"), (b"XXXX" + f[14][4:], "magic"),
                       (f[14][:4] + struct.pack("<I", 2) + f[14][8:], "version"),
                       (f[14][:12] + struct.pack("<I", 5) + f[14][16:], "head_layout")):
        bad = list(f)
        bad[14] = part
        expect_error("DecodeLayout", state.ingest_mooncake_bootstrap_frame, bad, name=what)
    bad = list(f)
    bad[14] = bad[14][:16 + 8] + struct.pack("<Q", 0) + bad[14][32:]   # num_layers 0
    with pytest.raises(kv.KvError):
        state.ingest_mooncake_bootstrap_frame(bad)
    bad = list(f)
    bad[14] = b""                                           # empty: no layout
    state.ingest_mooncake_bootstrap_frame(bad)
    assert state.decode_kv_args("s")["decode_layout"] is None
