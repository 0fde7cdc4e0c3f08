"""The C-ABI library: it loads, exports every symbol include/pbgdn.h declares,
and rejects bad arguments with status codes before any launch (no GPU needed)."""
import ctypes
import os
import re

import pytest

from pseudobrain_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "pbgdn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pbgdn_\w+)\s*\(", text)))


def test_header_declares_the_entry_points():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in declared_functions():
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name


def test_abi_version_and_status_strings():
    assert _lib.lib().pbgdn_abi_version() == _lib.ABI_VERSION == 14
    header = open(HEADER).read()
    assert re.search(r"#define PBGDN_ABI_VERSION (\d+)", header).group(1) == str(_lib.ABI_VERSION)
    assert _lib.status_string(0) == "ok"
    for code in (1, 2, 3, 4, 99):
        assert _lib.status_string(code)
    with pytest.raises(_lib.PbgdnError, match="status 2"):
        _lib.check(2, "x")


FAKE = 0x1000  # never dereferenced: every call below fails validation first


def chunk_call(**over):
    args = dict(q=FAKE, k=FAKE, v=FAKE, in_dtype=1, g=FAKE, beta=FAKE, beta_dtype=0, h0=None,
                ht=None, sdt=0, sidx=None, has_init=None, nstates=0, cu=None, nseq=1, o=FAKE, out_dtype=1, B=1, T=64, Hk=16, Hv=32, K=128,
                V=128, scale=0.1, chunk=64, ws=FAKE, ws_bytes=1 << 40, stream=None)
    args.update(over)
    return _lib.lib().pbgdn_chunk_fwd(*args.values())


def test_chunk_fwd_noalloc_rejects_calls_beyond_its_scratch():
    """The no-allocation prefill refuses, before touching any device, a call
    whose workspace would not fit its fixed scratch."""
    header = open(HEADER).read()
    assert re.search(r"#define PBGDN_NOALLOC_SCRATCH_BYTES \(64u << 20\)", header)
    lib = _lib.lib()
    assert lib.pbgdn_chunk_workspace_size(1, 32768, 32, 1, _lib.BF16) > _lib.NOALLOC_SCRATCH_BYTES
    args = dict(q=FAKE, k=FAKE, v=FAKE, in_dtype=1, g=FAKE, beta=FAKE, beta_dtype=0, h0=None, ht=None, sdt=0,
                sidx=None, has_init=None, nstates=0, cu=None, nseq=1, o=FAKE, out_dtype=1, B=1, T=32768, Hk=16,
                Hv=32, K=128, V=128, scale=0.1, chunk=64, stream=None)
    assert lib.pbgdn_chunk_fwd_noalloc(*args.values()) == _lib.ERR_SCRATCH
    assert "scratch" in _lib.status_string(_lib.ERR_SCRATCH)


def recurrent_call(**over):
    args = dict(q=FAKE, k=FAKE, v=FAKE, in_dtype=1, g=FAKE, beta=FAKE, beta_dtype=0, sin=FAKE,
                sout=FAKE, sdt=0, idx=None, nstates=1, o=FAKE, out_dtype=1, B=1, T=1, Hk=16, Hv=32, K=128,
                V=128, scale=0.1, policy=_lib.STATE_STREAM, stream=None)
    args.update(over)
    return _lib.lib().pbgdn_recurrent_fwd(*args.values())


@pytest.mark.parametrize("over,code", [
    (dict(in_dtype=5), _lib.ERR_INVALID_ARGUMENT),
    (dict(out_dtype=-1), _lib.ERR_INVALID_ARGUMENT),
    (dict(beta_dtype=2), _lib.ERR_INVALID_ARGUMENT),   # beta must be f32 or the input dtype
    (dict(Hv=24), _lib.ERR_INVALID_ARGUMENT),          # not a multiple of Hk
    (dict(T=-1), _lib.ERR_INVALID_ARGUMENT),
    (dict(nseq=2), _lib.ERR_INVALID_ARGUMENT),         # N must equal B without cu_seqlens
    (dict(cu=FAKE, B=2, nseq=2), _lib.ERR_INVALID_ARGUMENT),  # cu_seqlens needs B == 1
    (dict(q=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(chunk=32), _lib.ERR_UNSUPPORTED),
    (dict(K=96), _lib.ERR_UNSUPPORTED),
    (dict(K=512), _lib.ERR_UNSUPPORTED),
    (dict(K=256, in_dtype=0), _lib.ERR_UNSUPPORTED),  # 256-wide keys take 16-bit inputs
    (dict(K=256, V=80), _lib.ERR_UNSUPPORTED),        # and V a multiple of 32
    (dict(V=120), _lib.ERR_UNSUPPORTED),
    (dict(ws=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(ws=FAKE + 8), _lib.ERR_INVALID_ARGUMENT),     # workspace must be 16-byte aligned
    (dict(ws_bytes=1000), _lib.ERR_INVALID_ARGUMENT),  # smaller than pbgdn_chunk_workspace_size
    (dict(sdt=3), _lib.ERR_INVALID_ARGUMENT),           # state dtype code
    (dict(sidx=FAKE, nstates=-1), _lib.ERR_INVALID_ARGUMENT),
])
def test_chunk_fwd_rejects(over, code):
    assert chunk_call(**over) == code


def test_chunk_fwd_empty_is_ok():
    assert chunk_call(B=0, nseq=0) == _lib.OK


@pytest.mark.parametrize("over,code", [
    (dict(in_dtype=3), _lib.ERR_INVALID_ARGUMENT),
    (dict(Hk=0), _lib.ERR_INVALID_ARGUMENT),
    (dict(Hv=20), _lib.ERR_INVALID_ARGUMENT),
    (dict(sin=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(o=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(nstates=-1), _lib.ERR_INVALID_ARGUMENT),
    (dict(B=4, nstates=3), _lib.ERR_INVALID_ARGUMENT),  # without state_idx, slot b must exist
    (dict(sdt=4), _lib.ERR_INVALID_ARGUMENT),           # state dtype code
    (dict(sin=FAKE + 8), _lib.ERR_INVALID_ARGUMENT),    # a float32 state moves in 16-byte pieces
    (dict(sout=FAKE + 4, sdt=1), _lib.ERR_INVALID_ARGUMENT),  # a 16-bit state in 8-byte pieces
    (dict(v=FAKE + 8), _lib.ERR_INVALID_ARGUMENT),      # q, k, v are read in aligned words
    (dict(beta=FAKE + 2), _lib.ERR_INVALID_ARGUMENT),   # beta in 4-byte words
    (dict(K=48), _lib.ERR_UNSUPPORTED),
    (dict(V=512), _lib.ERR_UNSUPPORTED),
    (dict(B=70000, nstates=70000), _lib.ERR_UNSUPPORTED),
    (dict(policy=2), _lib.ERR_INVALID_ARGUMENT),        # PBGDN_STATE_STREAM or PBGDN_STATE_RESIDENT
    (dict(policy=-1, B=0), _lib.ERR_INVALID_ARGUMENT),
])
def test_recurrent_fwd_rejects(over, code):
    assert recurrent_call(**over) == code


def test_recurrent_fwd_empty_is_ok():
    assert recurrent_call(B=0) == _lib.OK
    assert recurrent_call(B=0, policy=_lib.STATE_RESIDENT) == _lib.OK


def test_state_policy_codes_match_the_header():
    header = open(HEADER).read()
    assert int(re.search(r"#define PBGDN_STATE_STREAM (\d+)", header).group(1)) == _lib.STATE_STREAM
    assert int(re.search(r"#define PBGDN_STATE_RESIDENT (\d+)", header).group(1)) == _lib.STATE_RESIDENT


@pytest.mark.parametrize("src,dst,nbytes", [
    (FAKE, FAKE + (1 << 20), 15),          # whole 16-byte pieces only
    (FAKE, FAKE + (1 << 20), -16),
    (FAKE, FAKE + (1 << 20), 1 << 31),     # at most 2 GiB - 16
    (FAKE + 8, FAKE + (1 << 20), 1024),    # 16-byte aligned
    (None, FAKE, 1024),
])
def test_stream_probe_rejects(src, dst, nbytes):
    assert _lib.lib().pbgdn_stream_probe(src, dst, nbytes, None) == _lib.ERR_INVALID_ARGUMENT


def test_stream_probe_empty_is_ok():
    assert _lib.lib().pbgdn_stream_probe(None, None, 0, None) == _lib.OK


def test_chunk_workspace_size():
    lib = _lib.lib()
    rec = 13 * 1024  # bytes per (64-token chunk, value head) record, 16-bit inputs
    rec32 = 19 * 1024  # float32 inputs: Tb's low part as well
    tail = 4096      # float32 inputs' range scale and its partial maxima
    # B*T tokens in N sequences: floor(B*T / 64) + N + 1 chunk records per value head
    for dt in (_lib.BF16, _lib.F16):
        assert lib.pbgdn_chunk_workspace_size(1, 32768, 32, 1, dt) == (512 + 2) * 32 * rec + tail
        assert lib.pbgdn_chunk_workspace_size(1, 262144, 32, 8, dt) == (4096 + 9) * 32 * rec + tail
        assert lib.pbgdn_chunk_workspace_size(4, 100, 2, 4, dt) == (6 + 5) * 2 * rec + tail
        assert lib.pbgdn_chunk_workspace_size(1, 0, 4, 1, dt) == 2 * 4 * rec + tail
    assert lib.pbgdn_chunk_workspace_size(1, 2048, 4, 1, _lib.F32) == (32 + 2) * 4 * rec32 + tail
    assert lib.pbgdn_chunk_workspace_size(-1, 10, 4, 1, _lib.BF16) == 0
    assert lib.pbgdn_chunk_workspace_size(1, 10, 0, 1, _lib.BF16) == 0
    assert lib.pbgdn_chunk_workspace_size(1, 10, 4, 1, 7) == 0  # dtype code


CH = 2 * 16 * 128 + 32 * 128  # q, k, v channels of the Qwen3-Next layer


def prologue_call(**over):
    args = dict(qkv=FAKE, qkv_stride=CH + 4096 + 64, decay=FAKE, decay_stride=CH + 4096 + 64, in_dtype=1,
                tail=FAKE, tail_out=FAKE + 4096, tail_dtype=0, w=FAKE, conv=4, a_log=FAKE, dt_bias=FAKE,
                q=FAKE, k=FAKE, v=FAKE, out_dtype=1, g=FAKE, beta=FAKE, B=1, T=64, Hk=16, Hv=32, K=128,
                V=128, l2=0, stream=None)
    args.update(over)
    return _lib.lib().pbgdn_prologue_fwd(*args.values())


def epilogue_call(**over):
    args = dict(o=FAKE, o_dtype=1, gate=FAKE, gate_stride=4096, gate_dtype=1, o_norm=FAKE, eps=1e-5,
                out=FAKE, out_dtype=1, B=1, T=64, Hv=32, V=128, stream=None)
    args.update(over)
    return _lib.lib().pbgdn_epilogue_fwd(*args.values())


@pytest.mark.parametrize("over,code", [
    (dict(in_dtype=3), _lib.ERR_INVALID_ARGUMENT),
    (dict(tail_dtype=-1), _lib.ERR_INVALID_ARGUMENT),
    (dict(l2=2), _lib.ERR_INVALID_ARGUMENT),
    (dict(Hv=24), _lib.ERR_INVALID_ARGUMENT),           # not a multiple of Hk
    (dict(conv=-1), _lib.ERR_INVALID_ARGUMENT),
    (dict(qkv_stride=CH - 8), _lib.ERR_INVALID_ARGUMENT),  # rows shorter than q, k, v
    (dict(qkv_stride=CH + 4), _lib.ERR_INVALID_ARGUMENT),  # not a multiple of 8
    (dict(decay_stride=63), _lib.ERR_INVALID_ARGUMENT),
    (dict(tail=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(w=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(qkv=FAKE + 8), _lib.ERR_INVALID_ARGUMENT),        # 16-byte alignment
    (dict(g=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(K=96), _lib.ERR_UNSUPPORTED),
    (dict(V=100), _lib.ERR_UNSUPPORTED),
    (dict(conv=5), _lib.ERR_UNSUPPORTED),
])
def test_prologue_fwd_rejects(over, code):
    assert prologue_call(**over) == code


def test_prologue_and_epilogue_empty_are_ok():
    assert prologue_call(B=0) == _lib.OK
    assert prologue_call(T=0) == _lib.OK
    assert epilogue_call(T=0) == _lib.OK


@pytest.mark.parametrize("over,code", [
    (dict(o_dtype=4), _lib.ERR_INVALID_ARGUMENT),
    (dict(out_dtype=-2), _lib.ERR_INVALID_ARGUMENT),
    (dict(eps=-1.0), _lib.ERR_INVALID_ARGUMENT),
    (dict(eps=float("nan")), _lib.ERR_INVALID_ARGUMENT),
    (dict(gate_stride=4000), _lib.ERR_INVALID_ARGUMENT),  # shorter than Hv * V
    (dict(gate=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(out=FAKE + 4), _lib.ERR_INVALID_ARGUMENT),
    (dict(V=96), _lib.ERR_UNSUPPORTED),
    (dict(V=256), _lib.ERR_UNSUPPORTED),
])
def test_epilogue_fwd_rejects(over, code):
    assert epilogue_call(**over) == code


def verify_call(**over):
    args = dict(q=FAKE, k=FAKE, v=FAKE, in_dtype=1, g=FAKE, beta=FAKE, beta_dtype=0, sin=FAKE,
                states=FAKE, sdt=0, idx=None, tidx=FAKE, nstates=8, o=FAKE, out_dtype=1, B=2, T=4, Hk=16, Hv=32,
                K=128, V=128, scale=0.1, stream=None)
    args.update(over)
    return _lib.lib().pbgdn_recurrent_verify_fwd(*args.values())


@pytest.mark.parametrize("over,code", [
    (dict(tidx=None), _lib.ERR_INVALID_ARGUMENT),        # the per-token slot table is required
    (dict(states=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(nstates=1), _lib.ERR_INVALID_ARGUMENT),        # without state_idx, slot b must exist
    (dict(sdt=-1), _lib.ERR_INVALID_ARGUMENT),
    (dict(states=FAKE + 2, sdt=2), _lib.ERR_INVALID_ARGUMENT),
    (dict(beta_dtype=2), _lib.ERR_INVALID_ARGUMENT),
    (dict(Hv=20), _lib.ERR_INVALID_ARGUMENT),
    (dict(K=48), _lib.ERR_UNSUPPORTED),
    (dict(B=70000, nstates=70000), _lib.ERR_UNSUPPORTED),
])
def test_recurrent_verify_fwd_rejects(over, code):
    assert verify_call(**over) == code


def test_recurrent_verify_fwd_empty_is_ok():
    assert verify_call(B=0) == _lib.OK
    assert verify_call(T=0) == _lib.OK


def decode_layer_call(**over):
    width = 2 * 16 * 128 + 2 * 32 * 128 + 64
    args = dict(z=FAKE, z_stride=width, in_dtype=1, conv_state=FAKE, conv_dtype=0, css=3 * CH, crs=CH, ccs=1,
                w=FAKE, conv=4, a_log=FAKE, dt_bias=FAKE, l2=0, state=FAKE, sdt=0, idx=None, nstates=64,
                o_norm=FAKE, eps=1e-5, hs=FAKE, out_dtype=0, B=64, Hk=16, Hv=32, K=128, V=128, scale=0.1,
                policy=_lib.STATE_STREAM, stream=None)
    args.update(over)
    return _lib.lib().pbgdn_decode_layer_fwd(*args.values())


@pytest.mark.parametrize("over,code", [
    (dict(z_stride=1000), _lib.ERR_INVALID_ARGUMENT),     # rows narrower than q|k|v|gate|a|b
    (dict(conv=5), _lib.ERR_INVALID_ARGUMENT),
    (dict(conv_state=None), _lib.ERR_INVALID_ARGUMENT),   # conv > 1 needs the tail pool
    (dict(w=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(l2=2), _lib.ERR_INVALID_ARGUMENT),
    (dict(eps=-1.0), _lib.ERR_INVALID_ARGUMENT),
    (dict(state=FAKE + 8), _lib.ERR_INVALID_ARGUMENT),    # a float32 state moves in 16-byte pieces
    (dict(nstates=10), _lib.ERR_INVALID_ARGUMENT),        # without state_idx, slot b must exist
    (dict(sdt=3), _lib.ERR_INVALID_ARGUMENT),
    (dict(Hv=24), _lib.ERR_INVALID_ARGUMENT),
    (dict(Hk=2, z_stride=1 << 20), _lib.ERR_UNSUPPORTED),  # 16 value heads per key head: more than 8
    (dict(K=96), _lib.ERR_UNSUPPORTED),
    (dict(V=256, z_stride=1 << 20), _lib.ERR_UNSUPPORTED),
    (dict(policy=7), _lib.ERR_INVALID_ARGUMENT),
])
def test_decode_layer_fwd_rejects(over, code):
    assert decode_layer_call(**over) == code


def test_decode_layer_fwd_empty_is_ok():
    assert decode_layer_call(B=0) == _lib.OK


def prologue_varlen_call(**over):
    args = dict(qkv=FAKE, qkv_stride=CH + 4096 + 64, decay=FAKE, decay_stride=CH + 4096 + 64, in_dtype=1,
                cu=FAKE, nseq=4, tail=FAKE, tail_out=FAKE, tail_dtype=0, tss=3 * CH, trs=CH, tcs=1, slots=None,
                has_init=None, nslots=4, w=FAKE, conv=4, a_log=FAKE, dt_bias=FAKE, q=FAKE, k=FAKE, v=FAKE,
                out_dtype=1, g=FAKE, beta=FAKE, T=64, Hk=16, Hv=32, K=128, V=128, l2=0, stream=None)
    args.update(over)
    return _lib.lib().pbgdn_prologue_varlen_fwd(*args.values())


@pytest.mark.parametrize("over,code", [
    (dict(cu=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(nseq=0), _lib.ERR_INVALID_ARGUMENT),           # tokens but no sequences
    (dict(tail=None), _lib.ERR_INVALID_ARGUMENT),        # conv > 1 needs the tail pool
    (dict(tcs=-1), _lib.ERR_INVALID_ARGUMENT),
    (dict(nslots=-1), _lib.ERR_INVALID_ARGUMENT),
    (dict(q=FAKE + 8), _lib.ERR_INVALID_ARGUMENT),       # 16-byte rows
    (dict(qkv_stride=CH + 4), _lib.ERR_INVALID_ARGUMENT),
    (dict(l2=3), _lib.ERR_INVALID_ARGUMENT),
    (dict(K=96), _lib.ERR_UNSUPPORTED),
    (dict(conv=5), _lib.ERR_UNSUPPORTED),
    (dict(nseq=70000), _lib.ERR_UNSUPPORTED),
])
def test_prologue_varlen_fwd_rejects(over, code):
    assert prologue_varlen_call(**over) == code


def test_prologue_varlen_fwd_empty_is_ok():
    assert prologue_varlen_call(T=0, nseq=0) == _lib.OK


def chunk_bwd_call(**over):
    args = dict(q=FAKE, k=FAKE, v=FAKE, in_dtype=1, g=FAKE, beta=FAKE, beta_dtype=0, h0=None, do=FAKE,
                do_dtype=1, dht=None, dq=FAKE, dk=FAKE, dv=FAKE, dg=FAKE, dbeta=FAKE, dh0=None, ws=FAKE,
                ws_bytes=1 << 40, B=1, T=64, Hk=16, Hv=32, K=128, V=128, scale=0.1, stream=None)
    args.update(over)
    return _lib.lib().pbgdn_chunk_bwd(*args.values())


@pytest.mark.parametrize("over,code", [
    (dict(in_dtype=3), _lib.ERR_INVALID_ARGUMENT),
    (dict(beta_dtype=-1), _lib.ERR_INVALID_ARGUMENT),
    (dict(do_dtype=5), _lib.ERR_INVALID_ARGUMENT),
    (dict(do_dtype=0), _lib.ERR_UNSUPPORTED),            # not q's dtype
    (dict(Hv=24), _lib.ERR_INVALID_ARGUMENT),            # not a multiple of Hk
    (dict(T=-1), _lib.ERR_INVALID_ARGUMENT),
    (dict(K=96), _lib.ERR_UNSUPPORTED),
    (dict(V=256), _lib.ERR_UNSUPPORTED),
    (dict(dq=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(do=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(ws=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(ws_bytes=1024), _lib.ERR_INVALID_ARGUMENT),    # smaller than the workspace size
    (dict(ws=FAKE + 4), _lib.ERR_INVALID_ARGUMENT),      # 16-byte alignment
    (dict(T=64 * 65536), _lib.ERR_UNSUPPORTED),          # more chunks than a grid axis holds
    (dict(B=32768), _lib.ERR_UNSUPPORTED),               # twice B rows of the scans' grid
    (dict(B=30000, Hk=65535, Hv=65535, T=64), _lib.ERR_UNSUPPORTED),  # the scans' 1-D grid past 2^31
])
def test_chunk_bwd_rejects_bad_arguments(over, code):
    assert chunk_bwd_call(**over) == code


def test_chunk_bwd_workspace_size():
    """Per (batch, value head, chunk): T (64 x 64), c and beta (64 each), dU0
    (64 x V) and the start state, end adjoint and J (K x V each) in float32;
    with GQA also dq and dk per value head; plus 256 bytes of slack."""
    size = _lib.lib().pbgdn_chunk_bwd_workspace_size
    per_record = 64 * 64 + 2 * 64 + 64 * 128 + 3 * 128 * 128
    assert size(2, 100, 4, 4, 128, 128) == 2 * 4 * 2 * per_record * 4 + 256
    assert size(1, 64, 2, 4, 128, 128) == (4 * per_record + 2 * 64 * 4 * 128) * 4 + 256
    assert size(1, 0, 1, 1, 64, 64) == 256
    assert size(-1, 64, 1, 1, 64, 64) == 0


def test_chunk_layer_fuses_rejects_and_declines_without_a_device_call():
    """The fusion query: -1 for arguments the layer prefill rejects, 0 for
    dtypes and widths the wide scan's epilogue does not take (decided before
    any device query)."""
    q = _lib.lib().pbgdn_chunk_layer_fuses
    assert q(9, _lib.BF16, _lib.F32, 4096, 1, 32, 128, 128) == -1       # dtype code
    assert q(_lib.BF16, _lib.BF16, _lib.F32, 4096, 1, 32, 128, 96) == -1  # epilogue widths 64, 128
    assert q(_lib.BF16, _lib.BF16, _lib.F32, 4096, -1, 32, 128, 128) == -1
    assert q(_lib.F32, _lib.F32, _lib.F32, 4096, 8, 32, 128, 128) == 0    # float32 inputs: two passes
    assert q(_lib.BF16, _lib.F16, _lib.F32, 4096, 8, 32, 128, 128) == 0   # gate in another dtype
    assert q(_lib.BF16, _lib.BF16, _lib.F32, 4096, 8, 32, 64, 128) == 0   # K = 64
