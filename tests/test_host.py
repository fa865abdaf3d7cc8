"""CPU-side tests: the C-ABI library loads and exports what include/nsn_hip.h
declares, host-side contracts (structural checks, byte accounting, split
heuristics), and that the product path neither imports the oracle nor falls
back to the CPU."""
import ast
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from nsn_amd import _lib, kernels, primitives
from nsn_amd.errors import IntegrityError
from tests.golden import inputs as gi

ROOT = Path(__file__).resolve().parent.parent


def header_functions():
    text = (ROOT / "include" / "nsn_hip.h").read_text()
    return set(re.findall(r"^\s*(?:const char \*|int64_t |int )\s*(nsn_\w+)\s*\(", text, re.M))


def test_library_exports_every_declared_symbol():
    declared = header_functions()
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    lib = _lib.lib()
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.nsn_version().startswith(b"nsn_hip")


def test_library_rejects_bad_arguments_without_gpu_work():
    lib = _lib.lib()
    # invalid bits / dtype / null pointers are rejected on the host before any launch
    assert lib.nsn_pack_codes(None, 10, 7, None, None, None) == _lib.NSN_EINVAL
    assert lib.nsn_unpack_codes(None, 10, 2, None, None) == _lib.NSN_EINVAL
    assert lib.nsn_encode_blocks(None, 9, 1, 1, 0, 0, 3, 0, 1, None, None, None, None, None, None, 1, 0, 0,
                                 None, None, None) == _lib.NSN_EINVAL
    assert lib.nsn_decode_attention(None, None) == _lib.NSN_EINVAL
    a = _lib.AttnArgs()
    a.batch, a.heads_q, a.heads_kv, a.bits = 1, 6, 4, 3          # 6 % 4 != 0
    assert lib.nsn_decode_attention(a, None) == _lib.NSN_EINVAL
    assert lib.nsn_attention_workspace_floats(16, 32, 8) == 16 * 32 * (8 * 132 + 1) == kernels.workspace_floats(16, 32, 8)
    # zero-size work is a no-op
    assert lib.nsn_pack_codes(None, 0, 3, None, None, None) == _lib.NSN_OK
    # prefill: the chunk's append needs both tails (fake, aligned, never dereferenced addresses)
    A = 1 << 20
    pa = _lib.PrefillArgs()
    pa.q, pa.ctx_len, pa.k_chunk, pa.v_chunk, pa.out = A, A, A, A, A
    pa.dtype, pa.batch, pa.heads_q, pa.heads_kv, pa.n_q, pa.bits = _lib.DTYPE_BF16, 1, 1, 1, 0, 3
    assert lib.nsn_prefill_attention(pa, None) == _lib.NSN_OK    # n_q = 0: nothing to do
    pa.n_q, pa.bits = 64, 4
    assert lib.nsn_prefill_attention(pa, None) == _lib.NSN_EINVAL
    pa.bits, pa.append = 3, 1
    assert lib.nsn_prefill_attention(pa, None) == _lib.NSN_EINVAL    # append without tails
    pa.k.tail, pa.k.tail_cap, pa.k.tail_dtype = A, 128, _lib.DTYPE_F16
    assert lib.nsn_prefill_attention(pa, None) == _lib.NSN_EINVAL    # the V tail is missing


def test_device_position_appends_reject_bad_arguments_without_gpu_work():
    """nsn_tail_append_to, nsn_tail_append_cast and nsn_rope_append validate on the host before any
    launch (fake, never dereferenced addresses stand in for device buffers)."""
    lib = _lib.lib()
    E, OK, F16 = _lib.NSN_EINVAL, _lib.NSN_OK, _lib.DTYPE_F16
    A = 1 << 20   # 16-byte aligned stand-in address

    def tail_to(rows=2, n=1, stride=1, cap=8, end=A, dtype=F16, k=A):
        return lib.nsn_tail_append_to(k, A, rows, n, stride, A, A, cap, end, dtype, A, None)
    assert tail_to(rows=-1) == E
    assert tail_to(n=3, stride=2) == E                 # row stride shorter than the tokens
    assert tail_to(n=9, stride=9, cap=8) == E          # more tokens than the tail holds
    assert tail_to(dtype=9) == E
    assert tail_to(end=None) == E                      # no device position
    assert tail_to(k=A + 8) == E                       # misaligned source
    assert tail_to(rows=0) == OK                       # empty: no work

    def cast(rows=2, n=1, stride=1, cap=8, off=0, sdt=_lib.DTYPE_BF16, dtype=F16, k=A):
        return lib.nsn_tail_append_cast(k, A, sdt, rows, n, stride, A, A, cap, off, dtype, None)
    assert cast(rows=-1) == E
    assert cast(n=3, stride=2) == E                    # row stride shorter than the tokens
    assert cast(n=4, stride=4, cap=8, off=5) == E      # past the tail's end
    assert cast(off=-1) == E
    assert cast(sdt=9) == E
    assert cast(dtype=_lib.DTYPE_F32) == E             # the tail is fp16 or bf16
    assert cast(k=A + 8) == E                          # misaligned source
    assert cast(k=None) == E
    assert cast(rows=0) == OK                          # empty: no work

    def rope(q_stride=8 * 128, kv_stride=2 * 128, cs=128, b=2, cap=8, end=A, offset=0, dtype=F16, q=A, tdt=F16):
        return lib.nsn_rope_append(q, A, A, q_stride, kv_stride, A, A, cs, b, 8, 2, A, A, A, cap, end, offset,
                                   dtype, tdt, A, None)
    assert rope(cs=64) == E                            # cos/sin rows overlap
    assert rope(q_stride=8 * 128 - 4) == E             # q rows overlap
    assert rope(kv_stride=2 * 128 + 2) == E            # 8-byte row alignment
    assert rope(dtype=_lib.DTYPE_F32) == E
    assert rope(tdt=_lib.DTYPE_F32) == E              # tails are fp16 or bf16
    assert rope(end=None, offset=8) == E               # host offset past the tail
    assert rope(cap=0) == E
    assert rope(q=A + 4) == E
    assert rope(q=None) == E
    assert rope(b=0) == OK


def test_planned_bytes_matches_reference_accounting():
    # loop_kv_pilot.py:407 and the paper's 3,724 B block (3072 + 640 + 12)
    assert primitives.planned_bytes((1, 1, 64, 128), 64, 4) == {"codes": 4096, "metadata": 640, "native": 0, "block_headers": 12}
    p = primitives.planned_bytes((1, 1, 64, 128), 64, 3)
    assert p["codes"] + p["metadata"] + p["block_headers"] == 3724
    with pytest.raises(IntegrityError):
        primitives.planned_bytes((1, 1, 64, 128), 65, 3)


def test_default_split_covers_context():
    for B, H, L in [(16, 8, 32768), (1, 8, 4133), (64, 4, 8192), (1, 1, 17)]:
        split, n = kernels.default_split(B, H, L)
        assert split % 64 == 0 and split * n >= L and split * (n - 1) < L


def _cpu_fixture(kind):
    """The reference's negative fixtures that fail structural checks (loop_kv_vf01_contract.py:98-120)."""
    a = gi.vf01_fixture(64, 65, "mixed_codes")
    t = lambda x, dt=torch.bfloat16: torch.from_numpy(x.view(np.int16)).view(dt) if x.dtype == np.uint16 else torch.from_numpy(x)
    q = t(a["q"])
    kt, vt = t(a["k_tail"]), t(a["v_tail"])
    g = {"codes": torch.from_numpy(a["k_codes"]), "metas": tuple(torch.from_numpy(a[f"k_meta{i}"]) for i in range(3)),
         "headers": torch.from_numpy(a["k_headers"])}
    vg = {"codes": torch.from_numpy(a["v_codes"]), "metas": tuple(torch.from_numpy(a[f"v_meta{i}"]) for i in range(3)),
          "headers": torch.from_numpy(a["v_headers"])}
    if kind == "q_shape":
        q = q[..., :127].contiguous()
    elif kind == "q_dtype":
        q = q.float()
    elif kind == "v_codes_short":
        vg["codes"] = vg["codes"][..., :-1].contiguous()
    elif kind == "v_meta_shape":
        vg["metas"] = (vg["metas"][0], vg["metas"][1][..., :127].contiguous(), vg["metas"][2])
    elif kind == "kv_length_mismatch":
        vt = torch.cat([vt, vt], 2)
    elif kind == "v_tail_noncontiguous":
        vt = vt.transpose(-1, -2).contiguous().transpose(-1, -2)
    elif kind == "k_codes_dtype":
        g["codes"] = g["codes"].to(torch.int16)
    elif kind == "empty_sequence":
        g = vg = None
        kt, vt = kt[:, :, :0], vt[:, :, :0]
    elif kind == "cpu_tensors":
        pass
    return g, kt, q, vg, vt


@pytest.mark.parametrize("kind", ["q_shape", "q_dtype", "v_codes_short", "v_meta_shape", "kv_length_mismatch",
                                  "v_tail_noncontiguous", "k_codes_dtype", "empty_sequence", "cpu_tensors"])
def test_structural_rejections(kind):
    data = _cpu_fixture(kind)
    with pytest.raises(IntegrityError):
        kernels.structural(*data)


def test_ops_refuse_cpu_tensors():
    x = torch.zeros(1, 64, 128)
    with pytest.raises(IntegrityError):
        primitives.nsn_encode(x, 3)
    with pytest.raises(IntegrityError):
        primitives.pack_codes(torch.zeros(8, dtype=torch.uint8), 3)


def test_product_path_never_imports_the_oracle():
    for path in (ROOT / "nsn_amd").rglob("*.py"):
        tree = ast.parse(path.read_text())
        for node in ast.walk(tree):
            if isinstance(node, ast.Import):
                assert not any(a.name.startswith("oracle") for a in node.names), path
            if isinstance(node, ast.ImportFrom):
                assert not (node.module or "").startswith("oracle"), path


def test_stream_cache_policy_matches_reference_formulas():
    """post_prefill / post_decode targets (loop_kv_pk01_cache.py:122-127), and
    the tail-length invariant they keep over a long token-by-token run."""
    from nsn_amd.stream_cache import decode_target, prefill_target
    for L in range(0, 1000):
        assert prefill_target(L) == max(0, ((L - 64) // 64) * 64)
    L, C = 8192, prefill_target(8192)
    assert L - C == 64
    for _ in range(5000):
        L += 1
        C = decode_target(L, C)
        assert C % 64 == 0 and 64 <= L - C < 128


def test_abi_struct_sizes_match_the_bindings():
    """The library reports the sizes of the argument structs it was built with;
    the ctypes mirrors must match them (a stale library whose nsn_attn_args
    differs from the bindings would read past the struct on the GPU)."""
    import ctypes
    from nsn_amd import _lib
    lib = _lib.lib()
    for which, st in enumerate((_lib.KVSide, _lib.AttnArgs, _lib.PrefillArgs, _lib.KScoreArgs)):
        assert lib.nsn_abi_sizeof(which) == ctypes.sizeof(st), st.__name__
    assert lib.nsn_abi_sizeof(4) == -1

    class Grown(ctypes.Structure):   # a layout with one more field than the library's
        _fields_ = _lib.AttnArgs._fields_ + [("extra", ctypes.c_void_p)]
    assert lib.nsn_abi_sizeof(1) != ctypes.sizeof(Grown)


def test_integration_binding_stubs_match_the_bindings():
    """The ctypes stubs INTEGRATION.md gives a maintainer (its python blocks'
    struct classes) have the package's field names, offsets and sizes."""
    import ctypes
    doc = (Path(__file__).resolve().parent.parent / "INTEGRATION.md").read_text()
    ns = {"ctypes": ctypes, "P": ctypes.c_void_p, "I32": ctypes.c_int, "I64": ctypes.c_int64}
    for block in re.findall(r"```python\n(.*?)```", doc, re.S):
        classes = re.findall(r"^class \w+\(ctypes\.Structure\):.*?\n(?:    .*\n)+", block, re.M)
        for c in classes:
            exec(c, ns)
    for name in ("KVSide", "AttnArgs", "PrefillArgs", "KScoreArgs"):
        assert name in ns, f"INTEGRATION.md has no {name} stub"
        doc_st, pkg_st = ns[name], getattr(_lib, name)
        assert [f[0] for f in doc_st._fields_] == [f[0] for f in pkg_st._fields_], name
        assert ctypes.sizeof(doc_st) == ctypes.sizeof(pkg_st), name
        for f, _ in doc_st._fields_:
            assert getattr(doc_st, f).offset == getattr(pkg_st, f).offset, (name, f)
