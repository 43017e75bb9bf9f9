"""CPU checks of the C ABI: the library loads, exports every symbol include/fam_hip.h
declares, the ctypes descriptor layouts match the C header, and argument validation
rejects bad calls before anything is launched (no GPU needed for any of this)."""
import ctypes as C
import os
import re
import subprocess
import tempfile

import pytest

from fam import _capi

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "fam_hip.h")


def _header_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(fam_\w+)\s*\(", src, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_capi.LIB_PATH):
        pytest.fail(f"{_capi.LIB_PATH} missing: run __graft_entry__.build() first")
    return _capi.load()


def test_exports_every_header_symbol(lib):
    names = _header_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), f"{n} declared in fam_hip.h but not exported"
    assert sorted(_capi.SIGNATURES) == names, "ctypes signatures must cover exactly the header's functions"
    out = subprocess.run(["nm", "-D", "--defined-only", _capi.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\sT\s(fam_\w+)", out))
    assert set(names) <= exported


def test_version(lib):
    assert lib.fam_version() == _capi.FAM_ABI_VERSION


def _c_offsets(struct: str, fields):
    prog = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    prog.append(f'printf("%zu\\n", sizeof({struct}));')
    for f in fields:
        prog.append(f'printf("%zu\\n", offsetof({struct}, {f}));')
    prog.append("return 0;}")
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "t.c")
        exe = os.path.join(d, "t")
        open(c, "w").write("\n".join(prog))
        subprocess.run(["gcc", "-std=c11", c, "-o", exe], check=True)
        vals = [int(v) for v in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    return vals[0], vals[1:]


@pytest.mark.parametrize("cls,cname", [(_capi.AttnDesc, "fam_attn_desc"), (_capi.GemmDesc, "fam_gemm_desc"),
                                       (_capi.RowopDesc, "fam_rowop_desc"), (_capi.CaeDesc, "fam_cae_desc"),
                                       (_capi.TinyDesc, "fam_tiny_desc"), (_capi.RowQ8Desc, "fam_rowq8_desc")])
def test_struct_layout_matches_header(cls, cname):
    fields = [f for f, _ in cls._fields_]
    size, offs = _c_offsets(cname, fields)
    assert C.sizeof(cls) == size
    for f, o in zip(fields, offs):
        assert getattr(cls, f).offset == o, f"{cname}.{f}"


def _err(lib):
    return lib.fam_last_error().decode()


def _tiny_desc(**kw):
    """A fam_tiny_desc at the CAE expert's shape with every pointer set to an aligned fake
    address (validation only; nothing is launched when a check fails)."""
    d = _capi.TinyDesc()
    dims = dict(batch=1, seq=8, hidden=32, heads=24, head_dim=128, ffn=256, action_dim=16, layers=30, steps=10,
                video_len=98, ctx_len=129, slice=0)
    dims.update({k: v for k, v in kw.items() if k in dims})
    for k, v in dims.items():
        setattr(d, k, v)
    d.eps, d.scale = 1e-6, 128 ** -0.5
    for i, (name, typ) in enumerate(_capi.TinyDesc._fields_):
        if typ is C.c_void_p:
            setattr(d, name, 4096 * (i + 1))
    A = d.heads * d.head_dim
    d.ctx_ld, d.video_rs, d.video_bs, d.mask_rs = 2 * A * d.layers, 3 * A, 0, 0
    d.ctx_emb_ld = 64
    d.video_mask = None
    for k, v in kw.items():
        if k not in dims:
            setattr(d, k, v)
    return d


def test_tiny_expert_validation(lib):
    """fam_tiny_expert refuses what its kernel does not cover before any launch (no GPU here:
    an accepted descriptor with an empty phase range returns FAM_OK without launching)."""
    f = lib.fam_tiny_expert
    assert f(C.byref(_tiny_desc()), 0, 0, None) == _capi.FAM_OK
    assert f(C.byref(_tiny_desc()), 0, 602, None) == _capi.FAM_ERR_INVALID_ARG      # past the final phase (2 L T)
    assert "phases" in _err(lib)
    assert f(C.byref(_tiny_desc(hidden=64)), 0, 0, None) == _capi.FAM_ERR_UNSUPPORTED
    assert f(C.byref(_tiny_desc(seq=17)), 0, 0, None) == _capi.FAM_ERR_INVALID_ARG
    assert f(C.byref(_tiny_desc(ffn=512)), 0, 0, None) == _capi.FAM_ERR_UNSUPPORTED
    assert f(C.byref(_tiny_desc(head_dim=12, heads=8)), 0, 0, None) == _capi.FAM_ERR_UNSUPPORTED
    # 16 heads of 8 in one 128-wide slice: 16 x 8 tokens = 128 attention columns > 32
    assert f(C.byref(_tiny_desc(heads=16, head_dim=8)), 0, 0, None) == _capi.FAM_ERR_UNSUPPORTED
    assert f(C.byref(_tiny_desc(gram=None)), 0, 0, None) == _capi.FAM_ERR_INVALID_ARG     # 24 slices need it
    assert f(C.byref(_tiny_desc(heads=4, head_dim=8, gram=None)), 0, 0, None) == _capi.FAM_OK   # one slice
    assert f(C.byref(_tiny_desc(qkv_w=4096 + 8)), 0, 0, None) == _capi.FAM_ERR_INVALID_ARG
    assert "aligned" in _err(lib)
    # a 32-wide slice reads the context K/V (ctx_ld), a wider one the context rows and factors
    assert f(C.byref(_tiny_desc(heads=4, head_dim=8, ctx_ld=100)), 0, 0, None) == _capi.FAM_ERR_INVALID_ARG
    assert f(C.byref(_tiny_desc(ctx_ld=100, ctxkv=None)), 0, 0, None) == _capi.FAM_OK
    assert f(C.byref(_tiny_desc(heads=4, head_dim=8, ctxkv=None)), 0, 0, None) == _capi.FAM_ERR_INVALID_ARG
    assert f(C.byref(_tiny_desc(ctx_emb_ld=30)), 0, 0, None) == _capi.FAM_ERR_INVALID_ARG
    assert f(C.byref(_tiny_desc(ck_wt=None)), 0, 0, None) == _capi.FAM_ERR_INVALID_ARG
    assert f(C.byref(_tiny_desc(ctx_rs=4096 + 8)), 0, 0, None) == _capi.FAM_ERR_INVALID_ARG
    assert f(C.byref(_tiny_desc(ctx_emb=4096 + 4)), 0, 0, None) == _capi.FAM_ERR_INVALID_ARG
    # fam_tiny_context validates the same descriptor; a 32-wide slice has nothing to compute
    assert lib.fam_tiny_context(C.byref(_tiny_desc(heads=4, head_dim=8)), None) == _capi.FAM_OK
    assert lib.fam_tiny_context(C.byref(_tiny_desc(ck_b=None)), None) == _capi.FAM_ERR_INVALID_ARG
    assert f(C.byref(_tiny_desc(video_rs=3072 * 3 + 4)), 0, 0, None) == _capi.FAM_ERR_INVALID_ARG
    assert f(C.byref(_tiny_desc(action_dim=40)), 0, 0, None) == _capi.FAM_ERR_UNSUPPORTED
    # context splits of the cross phases: one 32-wide slice (4 x 8 heads) over 1560 keys, one
    # batch row -> 7 splits of 7 blocks (each holds keys); none at 256 rows or over 100 keys;
    # forced counts capped; refused for several slices; part_x required once they are in use
    ks = lib.fam_tiny_key_splits
    c3 = dict(heads=4, head_dim=8, ctx_len=1560, video_len=0)
    assert ks(C.byref(_tiny_desc(**c3))) == 7
    assert ks(C.byref(_tiny_desc(**dict(c3, batch=256)))) == 1
    assert ks(C.byref(_tiny_desc(**dict(c3, ctx_len=100)))) == 1
    assert ks(C.byref(_tiny_desc(**dict(c3, key_splits=3)))) == 3
    assert ks(C.byref(_tiny_desc(**dict(c3, key_splits=50)))) == 7   # 8 splits of ceil(49 / 8) blocks: 7 hold keys
    assert ks(C.byref(_tiny_desc(ctx_len=1560, key_splits=3))) == -_capi.FAM_ERR_UNSUPPORTED
    assert f(C.byref(_tiny_desc(**dict(c3, part_x=None))), 0, 0, None) == _capi.FAM_ERR_INVALID_ARG
    assert f(C.byref(_tiny_desc(**dict(c3, part_x=4096 + 8))), 0, 0, None) == _capi.FAM_ERR_INVALID_ARG


def test_validation_rejects_before_launch(lib):
    # bad dims / alignment -> error codes, nothing launched (this host has no GPU)
    assert lib.fam_adaln(16, 1024, None, None, 0, 0, None, None, 32, 1024, 4, 4, 1020, 1e-6, None) == _capi.FAM_ERR_INVALID_ARG
    assert "dim" in _err(lib)
    assert lib.fam_adaln(16, 1024, 16, None, 0, 0, None, None, 32, 1024, 4, 4, 1024, 1e-6, None) == _capi.FAM_ERR_INVALID_ARG
    assert lib.fam_adaln(18, 1024, None, None, 0, 0, None, None, 32, 1024, 4, 4, 1024, 1e-6, None) == _capi.FAM_ERR_INVALID_ARG
    assert "aligned" in _err(lib)
    assert lib.fam_rmsnorm_rope(16, 64, 32, 64, 4, 4, 64, None, 1e-6, 64, 64, 32, 1, 12, None) == _capi.FAM_ERR_INVALID_ARG

    d = _capi.GemmDesc()
    d.a, d.w, d.out = 16, 32, 48
    d.M, d.N, d.K, d.lda, d.ldw, d.ldo, d.rows_per_batch = 32, 64, 7, 8, 8, 64, 32
    assert lib.fam_gemm(C.byref(d), None) == _capi.FAM_ERR_INVALID_ARG
    d.K, d.lda, d.ldw = 64, 64, 64
    d.prologue = 2  # AdaLN without shift/scale
    assert lib.fam_gemm(C.byref(d), None) == _capi.FAM_ERR_INVALID_ARG
    d.prologue = 0
    d.ldo = 32  # ldo < N
    assert lib.fam_gemm(C.byref(d), None) == _capi.FAM_ERR_INVALID_ARG
    d.ldo, d.gate = 64, 80  # a gate without a residual
    assert lib.fam_gemm(C.byref(d), None) == _capi.FAM_ERR_INVALID_ARG

    a = _capi.AttnDesc()
    a.q, a.k0, a.v0, a.o = 16, 32, 48, 64
    a.batch, a.heads, a.sq, a.sk0, a.head_dim = 1, 2, 4, 4, 48
    assert lib.fam_attention(C.byref(a), None) == _capi.FAM_ERR_UNSUPPORTED
    a.head_dim, a.q_rs = 64, 12
    assert lib.fam_attention(C.byref(a), None) == _capi.FAM_ERR_INVALID_ARG
    a.q_rs, a.mask_kind = 128, 1  # a mask kind without a mask
    assert lib.fam_attention(C.byref(a), None) == _capi.FAM_ERR_INVALID_ARG
    a.mask_kind = 7
    assert lib.fam_attention(C.byref(a), None) == _capi.FAM_ERR_INVALID_ARG

    a.mask_kind, a.num_splits = 0, 4  # key splits without partial buffers
    assert lib.fam_attention(C.byref(a), None) == _capi.FAM_ERR_INVALID_ARG
    assert lib.fam_attention_combine(C.byref(a), None) == _capi.FAM_ERR_INVALID_ARG
    a.num_splits = 65
    assert lib.fam_attention(C.byref(a), None) == _capi.FAM_ERR_INVALID_ARG

    # split-K partials: above 144 rows a K below 128 (off the large-M kernel), unaligned K,
    # misaligned partial buffer
    assert lib.fam_gemm_partial(16, 64, 32, 64, 48, 145, 64, 64, None) == _capi.FAM_ERR_UNSUPPORTED
    # 129..144 rows only on the streaming plan: not for a short K
    assert lib.fam_gemm_partial_splits(129, 64, 64) == 0
    assert lib.fam_gemm_partial(16, 64, 32, 64, 48, 129, 64, 64, None) == _capi.FAM_ERR_UNSUPPORTED
    assert lib.fam_gemm_partial_splits(129, 178176, 3072) == 1
    assert lib.fam_gemm_partial(16, 64, 32, 64, 48, 4, 64, 60, None) == _capi.FAM_ERR_INVALID_ARG
    assert lib.fam_gemm_partial(16, 64, 32, 64, 52, 4, 64, 64, None) == _capi.FAM_ERR_INVALID_ARG
    # the split plan of the action projections: >= 256 workgroups of 16 columns, fewest planes;
    # two-strip workgroups over 512-wide slices where they fill >= 192 workgroups without 1.5x
    # the planes (4096 x 1024, the real model's 9216 x 1024 q|k|v and 1024 x 3072 o)
    assert [lib.fam_gemm_partial_splits(32, n, k) for n, k in ((3072, 1024), (1024, 1024), (4096, 1024),
                                                              (1024, 4096), (7, 1024), (9216, 1024),
                                                              (1024, 3072))] == [2, 4, 2, 4, 8, 2, 6]
    assert lib.fam_gemm_partial_splits(0, 64, 64) == 0
    # above 144 rows the large-M kernel's planes: any shape with N % 4 == 0 and K % 64 == 0 (>= 128)
    # gets >= 1 plane; the head's N = 7 or a K tail does not.  1024 x 1024 x 4096 (config 1 at
    # B = 32, FFN down) is one round of 64 x 64 tiles with four K slots, unsplit (16.3 us measured
    # against 23.5 us for two planes); 2048 x 2048 x 8192 is split
    assert lib.fam_gemm_partial_splits(1024, 3072, 1024) >= 1 and lib.fam_gemm_partial_splits(1024, 1024, 4096) == 1
    assert lib.fam_gemm_partial_splits(2048, 2048, 8192) >= 2
    assert lib.fam_gemm_partial_splits(1024, 7, 1024) == 0 and lib.fam_gemm_partial_splits(1024, 1024, 1000) == 0
    assert lib.fam_gemm_partial(16, 64, 32, 64, 48, 1024, 7, 64, None) == _capi.FAM_ERR_UNSUPPORTED
    # cross-attention key splits: one launch up to 256 keys, about four 32-key blocks per split
    # beyond, at most 64 (config 1 at B=1 and 32, DiT4DiT over 2048 VLM tokens, a long context)
    assert [lib.fam_attention_key_splits(*a) for a in ((1, 16, 32, 1560, 64), (32, 16, 32, 1560, 64),
                                                      (1, 16, 16, 2048, 64), (1, 24, 32, 129, 128),
                                                      (1, 16, 32, 256, 64), (1, 16, 32, 257, 128),
                                                      (1, 16, 32, 100000, 64))] == [13, 13, 16, 1, 1, 3, 64]
    assert lib.fam_attention_key_splits(0, 16, 32, 1560, 64) == 0
    # the video prefill's 98-row projections: the streaming kernel (one round of 128-column
    # workgroups, whole 256-wide chunks per split) for FFN down / FFN up / q|k|v, 64-column
    # workgroups with 3 chunks per split for the 3072 x 3072 ones; the register kernel where
    # neither gives 3 chunks and the wide one would not fill the chip (98 x 4096 x 1024)
    assert [lib.fam_gemm_partial_splits(98, n, k) for n, k in ((3072, 14336), (14336, 3072), (9216, 3072),
                                                              (3072, 3072), (4096, 1024))] == [10, 2, 3, 4, 2]
    # above 64 rows the strides must stay below 2^23 elements (32-bit buffer offsets)
    assert lib.fam_gemm_partial(16, 3072, 32, 1 << 23, 48, 98, 64, 64, None) == _capi.FAM_ERR_UNSUPPORTED
    # ... and the activation span M * lda * 2 below 2^31 bytes: 144 rows at lda = 2^23 - 8 span
    # 2.4 GB although lda alone is below 2^23 (the out-of-range offsets would then read memory)
    assert lib.fam_gemm_partial(16, (1 << 23) - 8, 32, 3072, 48, 144, 178176, 3072, None) == _capi.FAM_ERR_UNSUPPORTED
    assert lib.fam_gemm_partial(16, (1 << 23) - 8, 32, 3072, 48, 129, 178176, 3072, None) == _capi.FAM_ERR_UNSUPPORTED

    r = _capi.RowopDesc()
    r.src, r.partials, r.splits, r.split_stride = _capi.FAM_ROWSRC_PARTIALS, 16, 2, 4 * 64
    r.M, r.N, r.out, r.ldo, r.rows_per_batch = 4, 64, 32, 64, 4
    r.norm = _capi.FAM_ROWNORM_ADALN  # AdaLN without a norm output / modulation
    assert lib.fam_rowop(C.byref(r), None) == _capi.FAM_ERR_INVALID_ARG
    r.nout, r.ldn = 48, 64
    assert lib.fam_rowop(C.byref(r), None) == _capi.FAM_ERR_INVALID_ARG
    assert "shift" in _err(lib)
    r.norm, r.nseg, r.seg_width = _capi.FAM_ROWNORM_RMS, 1, 6  # segment width not a multiple of 4
    assert lib.fam_rowop(C.byref(r), None) == _capi.FAM_ERR_INVALID_ARG
    # rows beyond one workgroup (4096 columns): only without normalisation on the vectorised path
    r.norm, r.nseg, r.N, r.ldo, r.split_stride = _capi.FAM_ROWNORM_NONE, 0, 20002, 20002, 4 * 20002
    assert lib.fam_rowop(C.byref(r), None) == _capi.FAM_ERR_INVALID_ARG    # N % 4 != 0
    assert "4096" in _err(lib)
    r.N, r.ldo, r.split_stride, r.ldn = 20000, 20000, 4 * 20000, 20000
    r.norm = _capi.FAM_ROWNORM_LAYERNORM
    assert lib.fam_rowop(C.byref(r), None) == _capi.FAM_ERR_INVALID_ARG    # a norm needs the whole row
    assert "4096" in _err(lib)
    r.norm = _capi.FAM_ROWNORM_NONE
    r.N, r.ldo, r.split_stride = 64, 64, 10  # partial planes overlap
    assert lib.fam_rowop(C.byref(r), None) == _capi.FAM_ERR_INVALID_ARG
    r.split_stride, r.src = 256, 9
    assert lib.fam_rowop(C.byref(r), None) == _capi.FAM_ERR_INVALID_ARG

    # grouped RMSNorm: groups >= 1 dividing the rows, weights present
    assert lib.fam_rmsnorm_grouped(16, 64, 32, 64, 9, 64, 48, 2, 1e-6, None) == _capi.FAM_ERR_INVALID_ARG
    assert lib.fam_rmsnorm_grouped(16, 64, 32, 64, 8, 64, 48, 0, 1e-6, None) == _capi.FAM_ERR_INVALID_ARG
    assert lib.fam_rmsnorm_grouped(16, 64, 32, 64, 8, 64, None, 2, 1e-6, None) == _capi.FAM_ERR_INVALID_ARG
    assert lib.fam_set_launch_events(16, None) == _capi.FAM_ERR_INVALID_ARG
    assert lib.fam_set_launch_events(None, None) == _capi.FAM_OK
    assert lib.fam_linear_smallk(16, 7, 0, 32, None, 48, 64, 4, 64, 65, None) == _capi.FAM_ERR_INVALID_ARG
    assert lib.fam_euler_step(16, 32, None, 48, 10, 10, None) == _capi.FAM_ERR_INVALID_ARG
    assert lib.fam_sinusoid(16, 32, 4, 7, None) == _capi.FAM_ERR_INVALID_ARG
    assert lib.fam_add_modulation(16, 32, 48, 2, 3, 12, None) == _capi.FAM_ERR_INVALID_ARG


def test_row_q8_and_mask_bias_validation(lib):
    """fam_row_q8 / fam_mask_bias refuse what their kernels do not take, before any launch."""
    q = _capi.RowQ8Desc()
    q.mode, q.x, q.ldx, q.y, q.ldy, q.s, q.M, q.D = _capi.FAM_Q8_ROW, 16, 64, 32, 64, 48, 4, 60
    assert lib.fam_row_q8(C.byref(q), None) == _capi.FAM_ERR_UNSUPPORTED          # D % 8 != 0
    q.D, q.ldx, q.ldy = 16392, 16392, 16392
    assert lib.fam_row_q8(C.byref(q), None) == _capi.FAM_ERR_UNSUPPORTED          # D past 16384
    assert "16384" in _err(lib)
    q.D, q.ldx, q.ldy = 64, 64, 64
    q.mode = 7
    assert lib.fam_row_q8(C.byref(q), None) == _capi.FAM_ERR_INVALID_ARG
    q.mode = _capi.FAM_Q8_LN_MOD                                                  # no shift / scale
    assert lib.fam_row_q8(C.byref(q), None) == _capi.FAM_ERR_INVALID_ARG
    q.shift, q.scale, q.eps = 64, 80, 1e-6
    q.x = 24                                                                      # x not 16-byte aligned
    assert lib.fam_row_q8(C.byref(q), None) == _capi.FAM_ERR_INVALID_ARG
    q.x, q.mode = 16, _capi.FAM_Q8_ADD_LN_MOD                                      # no x2 / xo
    assert lib.fam_row_q8(C.byref(q), None) == _capi.FAM_ERR_INVALID_ARG
    q.M = 0
    q.x2, q.ldx2, q.xo, q.ldxo = 96, 64, 112, 64
    assert lib.fam_row_q8(C.byref(q), None) == _capi.FAM_OK                       # no rows: nothing to do
    assert lib.fam_mask_bias(16, None, 0, 8, 106, 0, 16, 128, 0, None, None, None) == _capi.FAM_ERR_INVALID_ARG  # sb
    assert lib.fam_mask_bias(16, None, 0, 8, 106, 0, 4, 128, 0, 32, None, None) == _capi.FAM_ERR_INVALID_ARG   # MP < M
    assert lib.fam_mask_bias(16, 48, 30, 8, 106, 129, 16, 128, 256, 32, 64, None) == _capi.FAM_ERR_INVALID_ARG  # row stride < NS
    assert lib.fam_mask_bias(16, 48, 0, 8, 106, 129, 16, 128, 100, 32, 64, None) == _capi.FAM_ERR_INVALID_ARG  # NCP < NS


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(ImportError, match="build the HIP library"):
        _capi.load.__wrapped__(str(tmp_path / "nope.so")) if hasattr(_capi.load, "__wrapped__") else \
            _load_fresh(str(tmp_path / "nope.so"))


def _load_fresh(path):
    saved = _capi._lib
    _capi._lib = None
    try:
        return _capi.load(path)
    finally:
        _capi._lib = saved
