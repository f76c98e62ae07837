"""The kernels' manifest and ABI hashes (src/FuryKernel/Abi.hs,
Manifest.hs), and the native launch table's checks, on the CPU.

Pins: the reference's FNV-1a vectors (test/Test/FuryKernel/AbiTest.hs:33-36),
its ABI description text of rmsnorm (:43-53), its pinned ABI hash of scale
(:69-72, a hash of the whole canonical text, so a changed line or format
fails it), the C struct layout rule (:37-42), and its manifest of scale
(:73-122, rendered by the same writer)."""

import ctypes
import dataclasses

import pytest

from furykernel_amd import kernels as K
from furykernel_amd import manifest as M
from furykernel_amd import runtime


def abi(buffers, params, size, entry="k"):
    """A fk_kernel_abi built on the host, its strings kept alive on it."""
    keep = []

    def c(s):
        b = ctypes.c_char_p(s.encode())
        keep.append(b)
        return b

    bufs = (runtime.AbiBuffer * max(len(buffers), 1))()
    for i, (n, a, t, al) in enumerate(buffers):
        bufs[i].name, bufs[i].access, bufs[i].type, bufs[i].align = c(n).value, c(a).value, c(t).value, al
    prms = (runtime.AbiParam * max(len(params), 1))()
    for i, (n, t, o) in enumerate(params):
        prms[i].name, prms[i].type, prms[i].offset = c(n).value, c(t).value, o
    a = runtime.KernelAbi(entry.encode(), 0, len(buffers), bufs, len(params), prms, size, 0)
    a._keep = (keep, bufs, prms)
    return a


def test_fnv1a_reference_vectors():
    lib = runtime.library()
    for text, want in ((b"", 0xcbf29ce484222325), (b"a", 0xaf63dc4c8601ec8c), (b"foobar", 0x85944171f73967e8)):
        assert lib.fk_fnv1a64(text, len(text)) == want


def test_the_description_the_hash_covers():
    a = abi([("x", "read", "bf16", 16), ("w", "read", "bf16", 16), ("y", "write", "bf16", 16)],
            [("rows", "u32", 0), ("eps", "f32", 4)], 8)
    assert runtime.abi_description(a) == "\n".join([
        "abi 1", "buffer x read bf16 align 16", "buffer w read bf16 align 16", "buffer y write bf16 align 16",
        "param rows u32 at 0", "param eps f32 at 4", "params size 8"]) + "\n"


def test_the_pinned_abi_hash_of_scale():
    a = abi([("x", "read", "bf16", 16), ("y", "write", "bf16", 16)], [("n", "u32", 0), ("s", "f32", 4)], 8)
    assert runtime.library().fk_abi_hash(ctypes.byref(a)) == 0xe99ad54061a304ff
    renamed = abi([("x", "read", "bf16", 16), ("z", "write", "bf16", 16)], [("n", "u32", 0), ("s", "f32", 4)], 8)
    assert runtime.library().fk_abi_hash(ctypes.byref(renamed)) != 0xe99ad54061a304ff


def test_the_parameter_struct_is_laid_out_as_c_lays_it_out():
    class S(ctypes.Structure):
        _fields_ = [("a", ctypes.c_uint8), ("b", ctypes.c_float), ("c", ctypes.c_uint16), ("d", ctypes.c_uint32)]

    class T(ctypes.Structure):
        _fields_ = [("a", ctypes.c_float), ("b", ctypes.c_uint8)]
    assert [getattr(S, f).offset for f in "abcd"] == [0, 4, 8, 12] and ctypes.sizeof(S) == 16
    assert ctypes.sizeof(T) == 8


def test_the_manifest_of_scale_renders_as_the_reference_renders_it():
    text = M.render_json(M.kernel_manifest(
        "scale", 0xe99ad54061a304ff, 0x60c50bd78967a3d0, 64, "1u",
        [("x", "read", "bf16", 16, "$n"), ("y", "write", "bf16", 16, "$n")],
        [("n", "u32", 0, (1, 65536, 1)), ("s", "f32", 4, None)], 8, 0, target="T32"))
    assert text == "\n".join([
        "{", '  "format": "furykernel-manifest",', '  "version": 1,', '  "target": "T32",', '  "name": "scale",',
        '  "abi_hash": "0xe99ad54061a304ff",', '  "ir_hash": "0x60c50bd78967a3d0",', '  "threads": 64,',
        '  "groups": "1u",', '  "buffers": [', "    {", '      "name": "x",', '      "access": "read",',
        '      "type": "bf16",', '      "align": 16,', '      "extent": "$n"', "    },", "    {",
        '      "name": "y",', '      "access": "write",', '      "type": "bf16",', '      "align": 16,',
        '      "extent": "$n"', "    }", "  ],", '  "params": [', "    {", '      "name": "n",',
        '      "type": "u32",', '      "offset": 0,', '      "dim": {', '        "min": 1,',
        '        "max": 65536,', '        "multiple_of": 1', "      }", "    },", "    {", '      "name": "s",',
        '      "type": "f32",', '      "offset": 4', "    }", "  ],", '  "params_size": 8,',
        '  "threadgroup_memory": 0', "}"]) + "\n"


def _flat_fields(cls, base=0):
    out = []
    for name, ty in cls._fields_:
        off = getattr(cls, name).offset + base
        if isinstance(ty, type) and issubclass(ty, ctypes.Structure):
            out += _flat_fields(ty, off)
        elif hasattr(ty, "_length_"):
            out += [(f"{name}_{i}", off + 4 * i) for i in range(ty._length_)]
        else:
            out.append((name, off))
    return out


def test_every_kernel_is_in_the_manifest_with_the_bindings_abi():
    entries = set(runtime.manifest_entries())
    assert entries == set(K.ABIS)
    for entry, kabi in K.ABIS.items():
        a = runtime.abi_of(entry)
        assert [a.buffers[i].name.decode() for i in range(a.n_buffers)] == list(kabi.buffers), entry
        assert a.params_size == ctypes.sizeof(kabi.params), entry
        # the host binding's structs are the kernels' (fields and offsets)
        want = [(a.params[i].name.decode(), a.params[i].offset) for i in range(a.n_params)]
        got = _flat_fields(kabi.params)
        assert [o for _, o in got] == [o for _, o in want], entry
        assert a.abi_hash == runtime.library().fk_abi_hash(ctypes.byref(a))


def test_every_manifest_renders_and_parses():
    import json
    for entry in ("fk_step_gemv_f16_k2048_r2_p1_e3", "fk_step_attend", "fk_gemm_f16_qkv_rope", "fk_noop"):
        m = json.loads(M.render_json(M.manifest_of(entry)))
        assert m["format"] == "furykernel-manifest" and m["name"] == entry and m["target"] == "MI355X"
        assert m["abi_hash"] == M.hex64(runtime.abi_of(entry).abi_hash)


# The launch table's checks -----------------------------------------------------

def _spans(launch, specs, base=1 << 32):
    """Fake, distinct, aligned addresses of the right sizes for a launch's buffers."""
    out, at = [], base
    for b in K.ABIS[launch.entry].buffers:
        name = launch.bind.get(b)
        if name is None:
            out.append((0, 0))
        else:
            out.append((at, specs[name].nbytes))
            at += (specs[name].nbytes + 255) // 256 * 256
    return out


def _lowered_1b(options=None, wide=True):
    from furykernel_amd.lower import lower_plan
    from furykernel_amd.program.check import check_program
    from furykernel_amd.program.decoder import ONE_B, decoder_step
    from furykernel_amd.program.plan import PlanOptions, plan
    c = check_program(decoder_step(ONE_B, embed=True))
    return lower_plan(c, plan(options or PlanOptions(store_gelus=True), c), wide=wide)


def _check(launch, specs, **kw):
    from furykernel_amd.engine import params_struct
    runtime.launch_check(launch.entry, launch.groups, launch.threads, launch.lds_bytes,
                         kw.get("spans") or _spans(launch, specs), kw.get("params") or params_struct(launch),
                         kw.get("abi_hash"))


@pytest.mark.parametrize("wide", [False, True])
def test_the_launch_check_accepts_every_lowered_launch(wide):
    low = _lowered_1b(wide=wide)
    for L in low.launches:
        _check(L, low.buffers)


@pytest.mark.parametrize("wide,period,key", [(False, 6, 0), (False, 6, 3), (True, 5, 0), (True, 5, 2)])
def test_the_launch_check_refuses_the_probes_swapped_entries(wide, period, key):
    """Layer 0's gathering QKV (_p3) or O step (_e2) entry on a later layer's
    launch, whose token or res_token is unbound, is refused."""
    low = _lowered_1b(wide=wide)
    idx = [i for i in range(16 * period) if i % period == key]
    first = low.launches[idx[0]].entry
    for i in idx[1:]:
        L = dataclasses.replace(low.launches[i], entry=first)
        with pytest.raises(runtime.FkError, match="prologue|unbound"):
            _check(L, low.buffers)


def test_the_launch_check_refuses_wrong_hashes_sizes_and_short_buffers():
    from furykernel_amd.engine import params_struct
    low = _lowered_1b(wide=False)
    qkv = low.launches[6]
    good = runtime.abi_of(qkv.entry).abi_hash
    with pytest.raises(runtime.FkError, match="ABI hash"):
        _check(qkv, low.buffers, abi_hash=good ^ 1)
    spans = _spans(qkv, low.buffers)
    spans[1] = (spans[1][0], spans[1][1] - 2)  # w1 two bytes short
    with pytest.raises(runtime.FkError, match="w1 holds"):
        _check(qkv, low.buffers, spans=spans)
    spans = _spans(qkv, low.buffers)
    spans[0] = (spans[0][0] + 8, spans[0][1])  # w0 misaligned
    with pytest.raises(runtime.FkError, match="aligned"):
        _check(qkv, low.buffers, spans=spans)
    p = params_struct(qkv)
    p.pro_mode = 0
    with pytest.raises(runtime.FkError, match="its parameters say"):
        _check(qkv, low.buffers, params=p)
    att = low.launches[7]
    assert att.entry == "fk_step_attend"
    spans = _spans(att, low.buffers)
    spans[8] = (spans[8][0], spans[8][1] - 4)  # partials short
    with pytest.raises(runtime.FkError, match="partials holds"):
        _check(att, low.buffers, spans=spans)


def test_the_launch_check_refuses_wide_attention_and_combine_prologues_out_of_shape():
    from furykernel_amd.engine import params_struct
    low = _lowered_1b()
    att, o = low.launches[6], low.launches[7]
    assert att.entry == "fk_step_attend_wide" and o.params["pro_mode"] == K.PRO_COMBINE
    _check(att, low.buffers)
    _check(o, low.buffers)
    # a split that is not 32 positions a wavefront of the threadgroup
    p = params_struct(att)
    p.split = att.params["split"] // 2
    with pytest.raises(runtime.FkError):
        _check(att, low.buffers, params=p)
    # LDS short of what the wavefronts use
    short = dataclasses.replace(att, lds_bytes=att.lds_bytes - 4)
    with pytest.raises(runtime.FkError):
        _check(short, low.buffers)
    # more splits than the combine prologue takes
    p = params_struct(o)
    p.splits = K.COMBINE_SPLITS + 1
    with pytest.raises(runtime.FkError):
        _check(o, low.buffers, params=p)
    # partials shorter than the prologue reads
    spans = _spans(o, low.buffers)
    i = list(K.ABIS[o.entry].buffers).index("src")
    spans[i] = (spans[i][0], spans[i][1] - 4)
    with pytest.raises(runtime.FkError):
        _check(o, low.buffers, spans=spans)


def test_the_launch_check_takes_the_prefill_heads_keys_and_refuses_them_out_of_shape():
    from furykernel_amd.engine import params_struct
    from furykernel_amd.prefill import lower_prefill
    from furykernel_amd.program.check import check_program
    from furykernel_amd.program.decoder import SMALL_PREFILL, decoder_step
    from furykernel_amd.program.plan import PlanOptions, plan
    c = check_program(decoder_step(SMALL_PREFILL, name="prefill", position_bound=128))
    low = lower_prefill(c, plan(PlanOptions(sequence_rows=128), c), 256)
    for L in low.launches:
        _check(L, low.buffers)
    head, token = low.launches[-2:]
    assert (head.entry, token.entry) == ("fk_gemm_f16_store_keys", "fk_prefill_argmax_keys")
    # a GEMM's grid is its tiles, its LDS the ring
    for L in [l for l in low.launches if l.entry.startswith("fk_gemm_f16_")]:
        for bad in (dataclasses.replace(L, groups=L.groups + 1), dataclasses.replace(L, groups=L.groups - 1),
                    dataclasses.replace(L, lds_bytes=L.lds_bytes - 16)):
            with pytest.raises(runtime.FkError, match="threadgroup"):
                _check(bad, low.buffers)
        p = params_struct(L)
        p.k += 32   # k in pairs of steps of 32
        with pytest.raises(runtime.FkError, match="threadgroups"):
            _check(L, low.buffers, params=p)
    spans = _spans(head, low.buffers)
    i = list(K.ABIS[head.entry].buffers).index("keys")
    spans[i] = (spans[i][0], spans[i][1] - 8)  # one key short
    with pytest.raises(runtime.FkError, match="keys holds"):
        _check(head, low.buffers, spans=spans)
    p = params_struct(head)
    p.ldc[0] = p.first_col[1] + 256  # rows wider than the anchor's columns
    with pytest.raises(runtime.FkError, match="anchors"):
        _check(head, low.buffers, params=p)
    spans = _spans(token, low.buffers)
    spans[0] = (spans[0][0], spans[0][1] - 8)
    with pytest.raises(runtime.FkError, match="keys holds"):
        _check(token, low.buffers, spans=spans)
    p = params_struct(token)
    p.rows = 4 * token.groups + 1  # more rows than its waves
    with pytest.raises(runtime.FkError, match="rows"):
        _check(token, low.buffers, params=p)


def test_the_launch_check_takes_the_f16_prefill_attention_only_without_bf16_or_staged_rows():
    """The f16 form loads f16 ring rows straight into LDS: a launch of it
    with bf16 caches or staged rows is refused; the lowering gives those the
    staging form."""
    from furykernel_amd.engine import params_struct
    from furykernel_amd.prefill import lower_prefill
    from furykernel_amd.program.check import check_program
    from furykernel_amd.program.decoder import SMALL_PREFILL, decoder_step
    from furykernel_amd.program.plan import PlanOptions, plan
    c = check_program(decoder_step(SMALL_PREFILL, name="prefill", position_bound=128))
    low = lower_prefill(c, plan(PlanOptions(sequence_rows=128), c), 256)
    att = next(L for L in low.launches if L.entry.startswith("fk_prefill_attend"))
    assert att.entry == "fk_prefill_attend_f16_g2"
    _check(att, low.buffers)
    for field in ("cache_bf16", "staged"):
        p = params_struct(att)
        setattr(p, field, 1)
        if field == "staged":
            p.run_rows = 128
        with pytest.raises(runtime.FkError, match="bf16 caches"):
            _check(att, low.buffers, params=p)
    staged = check_program(decoder_step(SMALL_PREFILL, name="prefill"))
    low = lower_prefill(staged, plan(PlanOptions(sequence_rows=128), staged), 256, run_rows=128)
    assert {L.entry for L in low.launches if L.entry.startswith("fk_prefill_attend")} == {"fk_prefill_attend_g2"}


def test_the_launch_check_takes_the_paged_f16_attention_only_within_its_table_and_offsets():
    """The paged f16 form holds a block table of at most 256 entries in LDS and
    reads the pool at 32-bit offsets: larger tables, pools of 4 GiB or more,
    and bf16 pools are refused (the lowering gives those the other form)."""
    from furykernel_amd.engine import params_struct
    from furykernel_amd.prefill import lower_prefill
    from furykernel_amd.program.check import check_program
    from furykernel_amd.program.decoder import SMALL_PREFILL, decoder_step
    from furykernel_amd.program.plan import PlanOptions, plan
    c = check_program(decoder_step(SMALL_PREFILL, name="prefill", position_bound=128, paging=(64, 8)))
    low = lower_prefill(c, plan(PlanOptions(sequence_rows=128), c), 256, run_rows=128)
    att = next(L for L in low.launches if L.entry.startswith("fk_prefill_attend"))
    assert att.entry == "fk_prefill_attend_paged_f16_g2"
    _check(att, low.buffers)
    for field, value in (("cache_bf16", 1), ("table_len", 257), ("blocks", 1 << 20)):
        p = params_struct(att)
        setattr(p, field, value)
        with pytest.raises(runtime.FkError, match="bf16 caches|threadgroups"):
            _check(att, low.buffers, params=p)


def test_the_launch_check_refuses_prefill_attention_stores_and_lands_out_of_shape():
    """The ring prefill attention's grid is every (query block, kv head),
    its heads G to a kv head, its ring in blocks of 64 positions; the RoPE
    store and the landing of staged rows are one threadgroup a row.  Each
    is taken as lowered and refused with a grid, a group or a ring that
    would index past its buffers."""
    from furykernel_amd.engine import params_struct
    from furykernel_amd.prefill import lower_prefill
    from furykernel_amd.program.check import check_program
    from furykernel_amd.program.decoder import SMALL_PREFILL, decoder_step
    from furykernel_amd.program.plan import PlanOptions, plan
    # RoPE on some pairs (the separate store), positions up to the whole
    # ring (staged stores, landed after the attention)
    c = check_program(decoder_step(SMALL_PREFILL, name="prefill", rope_rotated=16))
    low = lower_prefill(c, plan(PlanOptions(sequence_rows=128), c), 256)
    by = {}
    for L in low.launches:
        _check(L, low.buffers)
        by.setdefault(L.entry, L)
    att, rope, land = by["fk_prefill_attend_g2"], by["fk_prefill_rope_store"], by["fk_prefill_land"]
    for L in (att, rope, land):
        for g in (L.groups + 1, L.groups - 1):
            with pytest.raises(runtime.FkError, match="threadgroups"):
                _check(dataclasses.replace(L, groups=g), low.buffers)
    p = params_struct(att)
    p.heads = p.heads + p.kv_heads   # a group of 3 launched as 2
    with pytest.raises(runtime.FkError, match="heads"):
        _check(att, low.buffers, params=p)
    p = params_struct(att)
    p.length = p.length - 32
    with pytest.raises(runtime.FkError, match="ring"):
        _check(att, low.buffers, params=p)
    with pytest.raises(runtime.FkError, match="threads"):
        _check(dataclasses.replace(att, threads=att.threads * 2), low.buffers)
    p = params_struct(rope)
    p.rotated = p.head_dim // 2 + 1
    with pytest.raises(runtime.FkError, match="pairs"):
        _check(rope, low.buffers, params=p)
    spans = _spans(rope, low.buffers)
    i = list(K.ABIS[rope.entry].buffers).index("qr")
    spans[i] = (spans[i][0], spans[i][1] - 2)
    with pytest.raises(runtime.FkError, match="qr holds"):
        _check(rope, low.buffers, spans=spans)
    p = params_struct(land)
    p.slots = 0
    with pytest.raises(runtime.FkError, match="slots"):
        _check(land, low.buffers, params=p)
