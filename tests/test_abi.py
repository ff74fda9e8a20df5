"""The C-ABI boundary, checked without a GPU.

* the built library loads and exports every function ``include/*.h`` declares;
* the ctypes structs have the C compiler's layout (sizeof / offsetof from a
  probe compiled with gcc against the header);
* host-side validation returns the documented codes and messages — these
  calls return before any HIP call, so they run on a machine without a GPU.
"""

from __future__ import annotations

import ctypes
import itertools
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

from ataraxos_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))

STRUCTS = {
    "AtxAttnParams": _lib.AttnParams,
    "AtxAttnBwdParams": _lib.AttnBwdParams,
    "AtxKqParams": _lib.KqParams,
    "AtxKqBwdParams": _lib.KqBwdParams,
    "AtxMhaParams": _lib.MhaParams,
    "AtxDecodeParams": _lib.DecodeParams,
    "AtxRolloutState": _lib.RolloutState,
}


def declared_functions() -> set[str]:
    names = set()
    for h in HEADERS:
        text = h.read_text()
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(atx_\w+)\s*\(", text, flags=re.M))
    return names


def test_header_declares_the_bound_entry_points():
    assert declared_functions() == set(_lib.ENTRY_POINTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.atx_abi_version() == _lib.ABI_VERSION


def test_header_constants_match_bindings():
    text = "".join(h.read_text() for h in HEADERS)
    consts = dict(re.findall(r"#define\s+(ATX_\w+)\s+\(?(-?\d+)\)?", text))
    assert int(consts["ATX_ABI_VERSION"]) == _lib.ABI_VERSION
    for name, val in [("ATX_OK", _lib.OK), ("ATX_ERR_INVALID_ARGUMENT", _lib.ERR_INVALID_ARGUMENT),
                      ("ATX_ERR_UNSUPPORTED", _lib.ERR_UNSUPPORTED), ("ATX_ERR_LAUNCH", _lib.ERR_LAUNCH),
                      ("ATX_ERR_ABI", _lib.ERR_ABI), ("ATX_DTYPE_FP32", _lib.DTYPE_FP32),
                      ("ATX_DTYPE_BF16", _lib.DTYPE_BF16), ("ATX_DTYPE_FP16", _lib.DTYPE_FP16),
                      ("ATX_KQ_OUT_PROBS", _lib.KQ_OUT_PROBS), ("ATX_KQ_OUT_LOGITS", _lib.KQ_OUT_LOGITS)]:
        assert int(consts[name]) == val, name


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_struct_layouts_match_c_compiler(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "ataraxos_attn.h"', '#include "ataraxos_rollout.h"',
             "int main(void) {"]
    for cname, py in STRUCTS.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'  printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    for line in filter(None, out):
        cname, field, value = line.split()
        py = STRUCTS[cname]
        want = ctypes.sizeof(py) if field == "size" else getattr(py, field).offset
        assert int(value) == want, f"{cname}.{field}: C {value}, ctypes {want}"


# --- validation without a GPU ------------------------------------------------


def _attn_params(**kw) -> _lib.AttnParams:
    p = _lib.AttnParams()
    p.abi_version = _lib.ABI_VERSION
    p.dtype = _lib.DTYPE_BF16
    p.batch, p.seq_q, p.seq_kv, p.num_heads, p.num_kv_heads, p.head_dim = 2, 100, 100, 6, 6, 64
    fake = 1 << 20  # never dereferenced: every case below fails validation first
    p.q = p.k = p.v = p.o = fake
    p.q_stride_b = p.k_stride_b = p.v_stride_b = p.o_stride_b = 100 * 384
    p.q_stride_s = p.k_stride_s = p.v_stride_s = p.o_stride_s = 384
    p.q_stride_h = p.k_stride_h = p.v_stride_h = p.o_stride_h = 64
    p.scale = 0.125
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def _expect(name, params, code, text):
    rc = _lib.call(name, params, None)
    assert rc == code, (rc, _lib.last_error())
    assert text in _lib.last_error()


def test_attention_validation_codes():
    lib = _lib.load()
    assert lib.atx_attn_fwd(None, None) == _lib.ERR_INVALID_ARGUMENT
    _expect("atx_attn_fwd", _attn_params(abi_version=99), _lib.ERR_ABI, "abi_version")
    _expect("atx_attn_fwd", _attn_params(dtype=7), _lib.ERR_INVALID_ARGUMENT, "dtype")
    _expect("atx_attn_fwd", _attn_params(batch=0), _lib.ERR_INVALID_ARGUMENT, "sizes")
    _expect("atx_attn_fwd", _attn_params(num_kv_heads=4), _lib.ERR_INVALID_ARGUMENT, "divisible")
    _expect("atx_attn_fwd", _attn_params(q=None), _lib.ERR_INVALID_ARGUMENT, "null")
    _expect("atx_attn_fwd", _attn_params(scale=0.0), _lib.ERR_INVALID_ARGUMENT, "scale")
    _expect("atx_attn_fwd", _attn_params(scale=float("nan")), _lib.ERR_INVALID_ARGUMENT, "scale")
    _expect("atx_attn_fwd", _attn_params(head_dim=8), _lib.ERR_UNSUPPORTED, "head_dim")
    _expect("atx_attn_fwd", _attn_params(head_dim=136), _lib.ERR_UNSUPPORTED, "head_dim")
    _expect("atx_attn_fwd", _attn_params(seq_kv=257), _lib.ERR_UNSUPPORTED, "seq_kv")
    _expect("atx_attn_fwd", _attn_params(q=(1 << 20) + 8), _lib.ERR_INVALID_ARGUMENT, "16-byte")
    _expect("atx_attn_fwd", _attn_params(k_stride_s=385), _lib.ERR_INVALID_ARGUMENT, "16-byte")
    _expect("atx_attn_fwd", _attn_params(o_stride_s=32), _lib.ERR_INVALID_ARGUMENT, "overlap")
    _expect("atx_attn_fwd", _attn_params(k_stride_s=-384), _lib.ERR_UNSUPPORTED, ">= 0")
    _expect("atx_attn_fwd", _attn_params(v_stride_s=1 << 26), _lib.ERR_UNSUPPORTED, "2 GiB")
    _expect("atx_attn_fwd", _attn_params(dropout_p=1.0), _lib.ERR_INVALID_ARGUMENT, "dropout_p")
    _expect("atx_attn_fwd", _attn_params(dropout_p=-0.1), _lib.ERR_INVALID_ARGUMENT, "dropout_p")
    _expect("atx_attn_fwd", _attn_params(dropout_p=float("nan")), _lib.ERR_INVALID_ARGUMENT, "dropout_p")
    _expect("atx_attn_fwd", _attn_params(dropout_p=0.1, head_dim=32, q_stride_h=32, k_stride_h=32, v_stride_h=32,
                                         o_stride_h=32), _lib.ERR_UNSUPPORTED, "dropout needs head_dim")


def _bwd_params(**kw) -> _lib.AttnBwdParams:
    p = _lib.AttnBwdParams()
    p.abi_version = _lib.ABI_VERSION
    p.dtype = _lib.DTYPE_BF16
    p.batch, p.seq_q, p.seq_kv, p.num_heads, p.num_kv_heads, p.head_dim = 2, 100, 100, 6, 6, 64
    fake = 1 << 20  # never dereferenced: every case below fails validation first
    for name in ("q", "k", "v", "o", "d_o", "dq", "dk", "dv"):
        setattr(p, name, fake)
    for name in ("q", "k", "v", "o", "do", "dq", "dk", "dv"):
        setattr(p, f"{name}_stride_b", 100 * 384)
        setattr(p, f"{name}_stride_s", 384)
        setattr(p, f"{name}_stride_h", 64)
    p.scale = 0.125
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_attention_backward_validation_codes():
    lib = _lib.load()
    assert lib.atx_attn_bwd(None, None) == _lib.ERR_INVALID_ARGUMENT
    _expect("atx_attn_bwd", _bwd_params(abi_version=99), _lib.ERR_ABI, "abi_version")
    _expect("atx_attn_bwd", _bwd_params(dtype=7), _lib.ERR_INVALID_ARGUMENT, "dtype")
    _expect("atx_attn_bwd", _bwd_params(seq_q=0), _lib.ERR_INVALID_ARGUMENT, "sizes")
    _expect("atx_attn_bwd", _bwd_params(num_kv_heads=4), _lib.ERR_INVALID_ARGUMENT, "divisible")
    _expect("atx_attn_bwd", _bwd_params(d_o=None), _lib.ERR_INVALID_ARGUMENT, "null")
    _expect("atx_attn_bwd", _bwd_params(dk=None), _lib.ERR_INVALID_ARGUMENT, "null")
    _expect("atx_attn_bwd", _bwd_params(scale=float("inf")), _lib.ERR_INVALID_ARGUMENT, "scale")
    _expect("atx_attn_bwd", _bwd_params(head_dim=24), _lib.ERR_UNSUPPORTED, "head_dim")
    _expect("atx_attn_bwd", _bwd_params(seq_kv=257), _lib.ERR_UNSUPPORTED, "256")
    _expect("atx_attn_bwd", _bwd_params(do_stride_s=385), _lib.ERR_INVALID_ARGUMENT, "16-byte")
    _expect("atx_attn_bwd", _bwd_params(dq=(1 << 20) + 8), _lib.ERR_INVALID_ARGUMENT, "16-byte")
    _expect("atx_attn_bwd", _bwd_params(v_stride_s=-384), _lib.ERR_UNSUPPORTED, ">= 0")
    _expect("atx_attn_bwd", _bwd_params(dv_stride_s=32), _lib.ERR_INVALID_ARGUMENT, "overlap")
    _expect("atx_attn_bwd", _bwd_params(dtype=_lib.DTYPE_FP32, head_dim=128, seq_q=256, seq_kv=256, **{
        f"{n}_stride_s": 768 for n in ("q", "k", "v", "o", "do", "dq", "dk", "dv")}), _lib.ERR_UNSUPPORTED, "LDS")
    _expect("atx_attn_bwd", _bwd_params(dropout_p=1.0), _lib.ERR_INVALID_ARGUMENT, "dropout_p")
    _expect("atx_attn_bwd", _bwd_params(dropout_p=0.2, head_dim=96, **{
        f"{n}_stride_h": 96 for n in ("q", "k", "v", "o", "do", "dq", "dk", "dv")}), _lib.ERR_UNSUPPORTED,
        "dropout needs head_dim")


def test_dropout_mask_validation_codes():
    lib = _lib.load()
    fake = 1 << 20  # never dereferenced: every case below fails validation first
    for args, text in [((0, 1, 4, 4, 0.1, 1, 0, fake), "sizes"), ((1, 1, 4, 4, 1.0, 1, 0, fake), "[0, 1)"),
                       ((1, 1, 4, 4, float("nan"), 1, 0, fake), "[0, 1)"), ((1, 1, 4, 4, 0.1, 1, 0, None), "NULL")]:
        assert lib.atx_dropout_mask(*args, None) == _lib.ERR_INVALID_ARGUMENT
        assert text in _lib.last_error()


def test_dropout_backward_plan():
    from ataraxos_amd import ops

    for d in ops.DROPOUT_HEAD_DIMS:
        for dt in (torch.bfloat16, torch.float32):
            for sq, h, hkv in ((101, 6, 6), (300, 8, 8), (64, 8, 2)):
                assert (ops.attention_backward_plan(d, sq, 101, h, hkv, dt, dropout=True)
                        == ops.attention_backward_plan(d, sq, 101, h, hkv, dt))
    assert ops.attention_backward_plan(32, 101, 101, 6, 6, torch.bfloat16, dropout=True) is None
    assert ops.attention_supported(48, 101, torch.float32, dropout=True)
    assert not ops.attention_supported(128, 101, torch.float32, dropout=True)


def test_backward_lds_rule_matches_python_predicate():
    """The library's LDS rule and ``ops.attention_backward_plan`` agree: every
    shape the plan refuses is refused by the library with the same byte
    count.  Shapes that pass are not called here, since their pointers are
    fake.  16-bit shapes all pass (queries are staged in blocks when needed);
    fp32 refuses head_dim >= 80 beyond 128 keys."""
    from ataraxos_amd import ops

    refused = 0
    for dtype, code in ((torch.bfloat16, _lib.DTYPE_BF16), (torch.float32, _lib.DTYPE_FP32)):
        for d in (16, 32, 48, 64, 80, 96, 112, 128):
            for sq, skv in ((100, 100), (256, 256), (40, 100), (256, 1), (1, 256), (200, 200), (129, 256), (600, 160)):
                plan = ops.attention_backward_plan(d, sq, skv, 4, 4, dtype)
                if plan is not None:
                    continue
                assert dtype == torch.float32 and d >= 80 and skv > 128, (d, sq, skv)
                strides = {f"{n}_stride_s": 2 * d for n in ("q", "k", "v", "o", "do", "dq", "dk", "dv")}
                p = _bwd_params(dtype=code, head_dim=d, seq_q=sq, seq_kv=skv, num_heads=1, num_kv_heads=1, **strides)
                assert _lib.call("atx_attn_bwd", p, None) == _lib.ERR_UNSUPPORTED
                want = ops._bwd_lds_bytes(d, 16, skv, True, 8)
                assert f"need {want} bytes of LDS" in _lib.last_error(), (d, sq, skv, _lib.last_error())
                refused += 1
    assert refused >= 8
    for args in ((64, 256, 256, 6, 6), (64, 100, 100, 6, 6), (128, 256, 256, 8, 2), (48, 101, 101, 8, 8)):
        assert ops.attention_backward_supported(*args, torch.bfloat16)
    assert ops.attention_backward_plan(64, 100, 100, 6, 6, torch.bfloat16) == {
        "loop": False, "key_chunks": 4, "query_block": 0, "lds": 66560}
    assert ops.attention_backward_plan(64, 100, 100, 8, 2, torch.bfloat16)["loop"]


def test_policy_validation_codes():
    p = _lib.KqParams()
    p.abi_version, p.dtype, p.batch, p.seq, p.dim = _lib.ABI_VERSION, _lib.DTYPE_BF16, 4, 100, 64
    p.q = p.k = p.out = 1 << 20
    p.q_stride_b = p.k_stride_b = 6400
    p.q_stride_s = p.k_stride_s = 64
    p.out_stride_b = 10000
    p.scale = 0.125
    for field, value, code, text in [
        ("out_mode", 5, _lib.ERR_INVALID_ARGUMENT, "out_mode"),
        ("seq", 129, _lib.ERR_UNSUPPORTED, "seq"),
        ("dim", 12, _lib.ERR_UNSUPPORTED, "dim"),
        ("scale", -1.0, _lib.ERR_INVALID_ARGUMENT, "scale"),
        ("out_stride_b", 9999, _lib.ERR_INVALID_ARGUMENT, "stride"),
    ]:
        saved = getattr(p, field)
        setattr(p, field, value)
        _expect("atx_kq_masked_softmax_fwd", p, code, text)
        setattr(p, field, saved)


def test_policy_backward_validation_codes():
    p = _lib.KqBwdParams()
    p.abi_version, p.dtype, p.batch, p.seq, p.dim = _lib.ABI_VERSION, _lib.DTYPE_BF16, 4, 100, 64
    p.out_mode = _lib.KQ_OUT_LOGITS
    p.q = p.k = p.dq = p.dk = p.grad = 1 << 20  # never dereferenced: every case fails validation
    p.q_stride_b = p.k_stride_b = p.dq_stride_b = p.dk_stride_b = 6400
    p.q_stride_s = p.k_stride_s = p.dq_stride_s = p.dk_stride_s = 64
    p.grad_stride_b = 10000
    p.scale = 0.125
    assert _lib.load().atx_kq_bwd(None, None) == _lib.ERR_INVALID_ARGUMENT
    for field, value, code, text in [
        ("abi_version", 99, _lib.ERR_ABI, "abi_version"),
        ("dtype", 9, _lib.ERR_INVALID_ARGUMENT, "dtype"),
        ("out_mode", 5, _lib.ERR_INVALID_ARGUMENT, "out_mode"),
        ("out_mode", _lib.KQ_OUT_PROBS, _lib.ERR_INVALID_ARGUMENT, "null"),  # probs mode needs probs
        ("seq", 129, _lib.ERR_UNSUPPORTED, "seq"),
        ("dim", 40, _lib.ERR_UNSUPPORTED, "dim"),
        ("dim", 144, _lib.ERR_UNSUPPORTED, "dim"),   # > 128: a multiple of 64
        ("dim", 4160, _lib.ERR_UNSUPPORTED, "dim"),
        ("scale", 0.0, _lib.ERR_INVALID_ARGUMENT, "scale"),
        ("grad_stride_b", 9999, _lib.ERR_INVALID_ARGUMENT, "stride"),
        ("dq_stride_s", 32, _lib.ERR_INVALID_ARGUMENT, "overlap"),
        ("k_stride_s", 68, _lib.ERR_INVALID_ARGUMENT, "16-byte"),
        ("q_stride_s", -64, _lib.ERR_UNSUPPORTED, ">= 0"),
    ]:
        saved = getattr(p, field)
        setattr(p, field, value)
        _expect("atx_kq_bwd", p, code, text)
        setattr(p, field, saved)


def test_fused_layer_validation_codes():
    p = _lib.MhaParams()
    p.abi_version, p.dtype, p.batch, p.seq, p.embed_dim, p.num_heads = _lib.ABI_VERSION, _lib.DTYPE_BF16, 4, 100, 384, 6
    p.x = p.w_q = p.w_k = p.w_v = p.w_o = p.y = 1 << 20  # never dereferenced: every case fails validation
    p.x_stride_b = p.y_stride_b = 100 * 384
    p.x_stride_s = p.y_stride_s = 384
    p.scale = 0.125
    assert _lib.load().atx_mha_fwd(None, None) == _lib.ERR_INVALID_ARGUMENT
    assert _lib.load().atx_mha_fwd_packed(None, None) == _lib.ERR_INVALID_ARGUMENT
    for (field, value, code, text), name in itertools.product([
        ("abi_version", 99, _lib.ERR_ABI, "abi_version"),
        ("dtype", _lib.DTYPE_FP32, _lib.ERR_UNSUPPORTED, "fp32"),
        ("embed_dim", 400, _lib.ERR_UNSUPPORTED, "head_dim"),
        ("num_heads", 3, _lib.ERR_UNSUPPORTED, "head_dim"),
        ("seq", 129, _lib.ERR_UNSUPPORTED, "seq"),
        ("w_o", None, _lib.ERR_INVALID_ARGUMENT, "null"),
        ("scale", -1.0, _lib.ERR_INVALID_ARGUMENT, "scale"),
        ("x_stride_s", 388, _lib.ERR_INVALID_ARGUMENT, "16-byte"),
        ("y_stride_s", 192, _lib.ERR_INVALID_ARGUMENT, "strides"),
    ], ("atx_mha_fwd", "atx_mha_fwd_packed")):
        saved = getattr(p, field)
        setattr(p, field, value)
        _expect(name, p, code, text)
        assert name in _lib.last_error()
        setattr(p, field, saved)
    p.embed_dim, p.num_heads, p.seq = 512, 8, 128
    p.x_stride_s = p.y_stride_s = 512
    _expect("atx_mha_fwd", p, _lib.ERR_UNSUPPORTED, "LDS")
    _expect("atx_mha_fwd_packed", p, _lib.ERR_UNSUPPORTED, "LDS")


def test_preln_block_validation_codes():
    """The pre-LN / residual fields of AtxMhaParams are checked before any HIP
    call: a bias without a weight, a residual flag other than 0/1, a negative
    or non-finite eps, misaligned LayerNorm vectors, and any shape outside
    the persistent kernel's (6 heads of 64 at 65..101 positions)."""
    p = _lib.MhaParams()
    p.abi_version, p.dtype, p.batch, p.seq, p.embed_dim, p.num_heads = _lib.ABI_VERSION, _lib.DTYPE_BF16, 4, 100, 384, 6
    p.x = p.w_q = p.w_k = p.w_v = p.w_o = p.y = 1 << 20  # never dereferenced: every case fails validation
    p.x_stride_b = p.y_stride_b = 100 * 384
    p.x_stride_s = p.y_stride_s = 384
    p.scale = 0.125
    p.ln_eps = 1e-5
    cases = [
        (dict(ln_bias=1 << 21), _lib.ERR_INVALID_ARGUMENT, "ln_bias without ln_weight"),
        (dict(residual=2), _lib.ERR_INVALID_ARGUMENT, "residual"),
        (dict(ln_weight=(1 << 21) + 2), _lib.ERR_INVALID_ARGUMENT, "16-byte"),
        (dict(ln_weight=1 << 21, ln_bias=(1 << 22) + 8), _lib.ERR_INVALID_ARGUMENT, "16-byte"),
        (dict(ln_weight=1 << 21, ln_eps=-1.0), _lib.ERR_INVALID_ARGUMENT, "ln_eps"),
        (dict(ln_weight=1 << 21, ln_eps=float("inf")), _lib.ERR_INVALID_ARGUMENT, "ln_eps"),
        (dict(residual=1, seq=64), _lib.ERR_UNSUPPORTED, "pre-LN / residual"),
        (dict(residual=1, seq=102), _lib.ERR_UNSUPPORTED, "pre-LN / residual"),
        (dict(ln_weight=1 << 21, num_heads=8), _lib.ERR_UNSUPPORTED, "pre-LN / residual"),
        (dict(residual=1, embed_dim=512, num_heads=8, x_stride_s=512, y_stride_s=512), _lib.ERR_UNSUPPORTED,
         "pre-LN / residual"),
    ]
    for fields, code, text in cases:
        saved = {k: getattr(p, k) for k in fields}
        for k, v in fields.items():
            setattr(p, k, v)
        for name in ("atx_mha_fwd", "atx_mha_fwd_packed"):
            _expect(name, p, code, text)
        for k, v in saved.items():
            setattr(p, k, v)


def test_workspace_entry_point_validation_codes():
    """atx_mha_fwd_ws validates the layer as atx_mha_fwd does, then the
    workspace (size, alignment, overlap), all before any HIP call."""
    lib = _lib.load()
    p = _lib.MhaParams()
    p.abi_version, p.dtype, p.batch, p.seq, p.embed_dim, p.num_heads = _lib.ABI_VERSION, _lib.DTYPE_BF16, 4, 100, 384, 6
    x, y = 1 << 30, 2 << 30
    p.x, p.y = x, y
    p.w_q, p.w_k, p.w_v, p.w_o = ((3 << 30) + i * (1 << 20) for i in range(4))
    p.x_stride_b = p.y_stride_b = 100 * 384
    p.x_stride_s = p.y_stride_s = 384
    p.scale = 0.125
    need = lib.atx_mha_workspace_bytes(384)
    assert need == 4 * 384 * 384 * 2 and lib.atx_mha_workspace_bytes(0) == 0
    ws = 4 << 30

    def expect(work, nbytes, code, text):
        rc = lib.atx_mha_fwd_ws(ctypes.byref(p), work, nbytes, None)
        assert rc == code, (rc, _lib.last_error())
        assert text in _lib.last_error() and "atx_mha_fwd_ws" in _lib.last_error()

    expect(None, need, _lib.ERR_INVALID_ARGUMENT, "NULL")
    expect(ws + 16, need, _lib.ERR_INVALID_ARGUMENT, "256-byte")
    expect(ws, need - 1, _lib.ERR_INVALID_ARGUMENT, "needs")
    expect(int(p.w_k) - 1024, need, _lib.ERR_INVALID_ARGUMENT, "overlaps a weight")
    expect(y + 4 * 100 * 384 * 2 - 256, need, _lib.ERR_INVALID_ARGUMENT, "overlaps x or y")
    expect(x - need + 256, need, _lib.ERR_INVALID_ARGUMENT, "overlaps x or y")
    p.seq = 129  # the layer itself is checked first
    expect(ws, need, _lib.ERR_UNSUPPORTED, "seq")
    assert lib.atx_mha_fwd_ws(None, ws, need, None) == _lib.ERR_INVALID_ARGUMENT


def test_output_and_alignment_helpers():
    """ops._check_out refuses outputs the ABI cannot describe (wrong shape or
    dtype, a strided last dim, misaligned rows); ops._aligned_rows copies a
    contiguous view that starts at a misaligned address."""
    from ataraxos_amd import ops

    dev = torch.device("cpu")
    good = torch.empty(2, 3, 4, 16, dtype=torch.bfloat16)
    ops._check_out("t", good, (2, 3, 4, 16), torch.bfloat16, dev)
    for bad, text in [
        (torch.empty(2, 3, 4, 8, dtype=torch.bfloat16), "out must be"),
        (torch.empty(2, 3, 4, 16, dtype=torch.float32), "out must be"),
        (torch.empty(2, 3, 4, 32, dtype=torch.bfloat16)[..., ::2], "contiguous last dim"),
        (torch.empty(2 * 3 * 4 * 16 + 1, dtype=torch.bfloat16)[1:].view(2, 3, 4, 16), "16-byte"),
    ]:
        with pytest.raises(ValueError, match=text):
            ops._check_out("t", bad, (2, 3, 4, 16), torch.bfloat16, dev)
    base = torch.arange(1 + 4 * 64, dtype=torch.bfloat16)
    mis = base[1:].view(4, 64)
    assert mis.is_contiguous() and mis.data_ptr() % 16 != 0
    fixed = ops._aligned_rows(mis)
    assert fixed.data_ptr() % 16 == 0 and torch.equal(fixed, mis)
    strided = torch.arange(4 * 128, dtype=torch.bfloat16).view(4, 128)[:, ::2]
    fixed = ops._aligned_rows(strided)
    assert fixed.stride(-1) == 1 and torch.equal(fixed, strided)
    assert ops._aligned_rows(good) is good


def test_decoders_refuse_networks_they_do_not_restate():
    """SetupDecoder needs causal blocks; BeliefDecoder needs pre-LN decoder
    layers (its per-row step applies the norms first)."""
    from ataraxos_amd import BeliefDecoder, SetupDecoder
    from tests._netlike import BeliefLike, SetupLike

    net = SetupLike(depth=2, dim=64, heads=2, ff=64)
    net.blocks.blocks[1].attn.causal = False
    with pytest.raises(ValueError, match="not causal"):
        SetupDecoder(net, 2, capacity=4)
    bnet = BeliefLike(channels=4, dim=64, heads=2, ff=64, enc_depth=1, dec_layers=2)
    bnet.decoder.layers[1].norm_first = False
    with pytest.raises(ValueError, match="norm_first"):
        BeliefDecoder(bnet, torch.zeros(2, 4, 10, 10), torch.ones(2, 100, dtype=torch.bool))


def test_weight_pack_validation_codes():
    """atx_mha_pack_weight rejects every bad argument before touching memory."""
    lib = _lib.load()
    a, b = 1 << 20, 1 << 24  # never dereferenced
    for args, code, text in [
        ((_lib.DTYPE_FP32, 384, a, b), _lib.ERR_UNSUPPORTED, "16-bit"),
        ((9, 384, a, b), _lib.ERR_INVALID_ARGUMENT, "dtype"),
        ((_lib.DTYPE_BF16, 48, a, b), _lib.ERR_INVALID_ARGUMENT, "multiple of 32"),
        ((_lib.DTYPE_BF16, 8192, a, b), _lib.ERR_INVALID_ARGUMENT, "multiple of 32"),
        ((_lib.DTYPE_BF16, 384, None, b), _lib.ERR_INVALID_ARGUMENT, "null"),
        ((_lib.DTYPE_BF16, 384, a + 8, b), _lib.ERR_INVALID_ARGUMENT, "aligned"),
        ((_lib.DTYPE_BF16, 384, a, a + 1024), _lib.ERR_INVALID_ARGUMENT, "overlap"),
    ]:
        assert lib.atx_mha_pack_weight(*args, None) == code, args
        assert text in _lib.last_error(), (args, _lib.last_error())


def test_decode_validation_codes():
    p = _lib.DecodeParams()
    p.abi_version, p.dtype, p.batch, p.num_heads, p.num_kv_heads, p.head_dim = _lib.ABI_VERSION, _lib.DTYPE_BF16, 4, 8, 8, 64
    p.kv_capacity, p.kv_len = 40, 41
    p.q = p.k_cache = p.v_cache = p.o = 1 << 20
    p.scale = 0.125
    _expect("atx_attn_decode_fwd", p, _lib.ERR_INVALID_ARGUMENT, "kv_len")
    p.kv_len = 10
    p.k_new = 1 << 20
    _expect("atx_attn_decode_fwd", p, _lib.ERR_INVALID_ARGUMENT, "together")
    p.k_new = None
    p.head_dim = 12
    _expect("atx_attn_decode_fwd", p, _lib.ERR_UNSUPPORTED, "multiple")


def test_error_text_is_per_call():
    _expect("atx_attn_fwd", _attn_params(head_dim=8), _lib.ERR_UNSUPPORTED, "head_dim")
    _expect("atx_attn_fwd", _attn_params(dtype=9), _lib.ERR_INVALID_ARGUMENT, "dtype")
    assert "head_dim" not in _lib.last_error()


def test_missing_library_raises_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setenv("ATARAXOS_AMD_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(_lib.AtxError, match="not found"):
        _lib.load()
    assert not _lib.available()


def test_rollout_validation_codes():
    """atx_rollout_*: ABI mismatch, negative and zero game counts, null
    arrays; none of these reaches a launch."""
    lib = _lib.load()
    st = _lib.RolloutState()
    st.abi_version = _lib.ABI_VERSION
    st.n_games = 0
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced
    for name, args in (("atx_rollout_apply", (fake,)), ("atx_rollout_legal_mask", (fake,)),
                       ("atx_rollout_infostate", (fake,)), ("atx_rollout_hash", (fake,)),
                       ("atx_rollout_reset", (fake, fake, 1))):
        fn = getattr(lib, name)
        assert fn(ctypes.byref(st), *args, None) == _lib.OK, name  # zero games: nothing to do
        st.abi_version = 0
        assert fn(ctypes.byref(st), *args, None) == _lib.ERR_ABI
        assert "abi_version" in _lib.last_error()
        st.abi_version, st.n_games = _lib.ABI_VERSION, -1
        assert fn(ctypes.byref(st), *args, None) == _lib.ERR_INVALID_ARGUMENT
        st.n_games = 4  # arrays still null
        assert fn(ctypes.byref(st), *args, None) == _lib.ERR_INVALID_ARGUMENT
        assert "null" in _lib.last_error()
        st.n_games = 0
    assert lib.atx_rollout_hello(None, -1, None) == _lib.ERR_INVALID_ARGUMENT
    assert lib.atx_rollout_hello(None, 0, None) == _lib.OK
