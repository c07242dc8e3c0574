"""C-ABI and host-logic tests that need no GPU: the library loads and exports every symbol
include/fracture_hip.h declares; the host helpers reproduce the oracle bit for bit; the
TurboQuant configuration mirrors turboquant.rs; argument checking fails on the host.
"""
import subprocess

import numpy as np
import pytest

import oracle
from fracture_amd import _lib
from fracture_amd import turboquant as tq


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    declared = _lib.header_symbols()
    assert len(declared) > 60
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                        text=True, check=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if " T " in line}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    for s in declared:
        assert getattr(lib, s) is not None
    # the Python binding declares a signature for each of them
    assert set(declared) <= set(_lib.SIGNATURES), set(declared) - set(_lib.SIGNATURES)


def test_reference_launcher_names_are_covered():
    # one fhip_launch_* per launch_* symbol of backends/fracture-cuda/src/ffi.rs:141-274
    ref = ["rmsnorm", "rope", "silu_mul", "embedding", "add", "turboquant_compress",
           "turboquant_decompress", "attention_paged_tq", "attention", "paged_attention"]
    for name in ref:
        assert f"fhip_launch_{name}" in _lib.header_symbols()


def test_version():
    assert b"gfx950" in _lib.load().fhip_version()


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 8])
def test_codebook_equals_oracle(bits):
    c, b = tq.codebook(128, bits)
    oc, ob, _ = oracle.lloyd_max(128, bits)
    assert np.array_equal(c, oc) and np.array_equal(b, ob)


@pytest.mark.parametrize("d,seed", [(16, 42), (128, 42), (128, 542), (64, 5042)])
def test_rotation_equals_oracle(d, seed):
    assert np.array_equal(tq.rotation_matrix(d, seed), oracle.rotation(d, seed))


def test_rope_freqs_equal_oracle():
    for hd, theta in [(128, 500000.0), (32, 500000.0), (64, 10000.0)]:
        assert np.array_equal(tq.rope_freqs(hd, theta), oracle.rope_freqs(hd, theta))


def test_rotation_seeds():
    assert tq.rotation_seeds(42, 0) == (42, 542)
    assert tq.rotation_seeds(42, 5) == (5042, 5542)


# TurboQuantConfig (turboquant.rs:440-800 tests)
def test_config_default_and_layers():
    cfg = tq.TurboQuantConfig()
    assert (cfg.key_bits, cfg.value_bits, cfg.protected_bits, cfg.protected_layers,
            cfg.residual_tokens, cfg.seed) == (4, 2, 8, 0, 0, 42)
    cfg.validate()
    p = tq.TurboQuantConfig(protected_layers=2)
    assert [p.key_bits_for_layer(l, 32) for l in (0, 1, 2, 15, 29, 30, 31)] == [8, 8, 4, 4, 4, 8, 8]
    assert [p.value_bits_for_layer(l, 32) for l in (0, 15, 31)] == [8, 2, 8]
    assert tq.TurboQuantConfig(protected_layers=20).is_protected(15, 32)
    assert tq.TurboQuantConfig(protected_layers=1).is_protected(0, 1)
    assert tq.TurboQuantConfig().distinct_bit_widths() == [2, 4]
    assert p.distinct_bit_widths() == [2, 4, 8]
    with pytest.raises(ValueError):
        tq.TurboQuantConfig(key_bits=5).validate()


def test_config_sizes():
    C = tq.TurboQuantConfig
    assert [C.packed_dim_per_head(128, b) for b in (4, 2, 8, 3)] == [64, 32, 128, 48]
    assert C.packed_dim_per_head(96, 4) == 48 and C.packed_dim_per_head(5, 4) == 3
    assert C.bytes_per_block_layer(8, 128, 4, 2) == 12800
    assert C.bytes_per_block_layer(8, 128, 8, 8) == 33280
    assert C().bytes_per_block_total(32, 8, 128) == 12800 * 32
    cfg = C(protected_layers=4)
    assert cfg.bytes_per_block_total(32, 8, 128) == 8 * 33280 + 24 * 12800
    per = C().bytes_per_block_total(32, 8, 128)
    assert C().compute_num_blocks(3 * per, 0, 32, 8, 128) == 3
    assert C().compute_num_blocks(4 * per - 1, 0, 32, 8, 128) == 3
    assert C().compute_num_blocks(1000, 2000, 32, 8, 128) == 0


def test_raw_launchers_reject_bad_arguments_on_host():
    lib = _lib.load()
    # invalid sizes are refused before any launch (hipErrorInvalidValue = 1)
    assert lib.fhip_launch_rmsnorm(None, None, None, 1e-5, -1, 4, None) == 1
    assert lib.fhip_launch_turboquant_compress(None, None, None, None, None, 1, 1, 128, 16, 4, 63,
                                               None) == 1  # wrong packed dim
    assert lib.fhip_launch_turboquant_compress(None, None, None, None, None, 1, 1, 128, 32, 4, 64,
                                               None) == 1  # 32 levels > 2^4
    assert lib.fhip_launch_tq_quantize_pack(None, None, 16, 9, None, 1, 128, 144, None) == 1
    # plans: head_dim 128 only, a valid codebook, an output handle; launchers need a plan
    import ctypes

    h = ctypes.c_void_p(1)
    assert lib.fhip_tq_plan_create(1, 1, 16, 4, 64, None, ctypes.byref(h)) == 1
    assert not h.value  # cleared on failure
    assert lib.fhip_tq_plan_create(1, 1, 17, 4, 128, None, ctypes.byref(h)) == 1
    assert lib.fhip_tq_plan_create(None, 1, 16, 4, 128, None, ctypes.byref(h)) == 1
    assert lib.fhip_tq_plan_create(1, 1, 16, 4, 128, None, None) == 1
    assert lib.fhip_launch_tq_compress_planned(None, 1, 1, 1, 4, 8, None) == 1
    assert lib.fhip_launch_tq_dequant_planned(None, 1, 1, 1, 4, 8, None) == 1
    lib.fhip_tq_plan_destroy(None)  # no-op
    # zero-size work is a no-op success
    assert lib.fhip_launch_add(None, None, None, 0, None) == 0
    assert lib.fhip_rows_workspace_bytes(64, 128256) == 64 * 32 * 32
    # FP16 paged attention: head_dim 1 to 256, heads divisible, context bound
    assert lib.fhip_launch_paged_attention(1, 1, 1, 1, 1, 1, 8, 2, 264, 16, 0, 1, None) == 1
    assert lib.fhip_launch_paged_attention(1, 1, 1, 1, 1, 1, 8, 2, 0, 16, 0, 1, None) == 1
    assert lib.fhip_launch_paged_attention(1, 1, 1, 1, 1, 1, 6, 4, 128, 16, 0, 1, None) == 1
    assert lib.fhip_launch_paged_attention(1, 1, 1, 1, 1, -1, 8, 2, 128, 16, 0, 1, None) == 1
    assert lib.fhip_launch_paged_attention(None, None, None, None, None, 0, 8, 2, 128, 16, 0, 1,
                                           None) == 0  # no tokens: nothing to do
    assert lib.fhip_launch_attention_paged_decode(1, 1, 1, 1, 1, 1 << 17, 1, 1, 1, 1, 1, 8, 2, 128,
                                                  1, None) == 1  # 2M positions > the 1M bound
    # batched decode: a block table of zero width (a batch of empty sequences only) is refused
    i64 = ctypes.c_int64
    assert lib.fhip_launch_attention_paged_decode(1, 1, 1, 1, 2, 0, 1, 1, 1, i64(1), i64(1), 8, 2,
                                                  128, 1, None) == 1
    assert lib.fhip_launch_attention_tq_decode(1, 1, 1, 1, 2, 0, 4, 1, 1, 1, 1, i64(4096), i64(256),
                                               i64(4096), i64(256), 1, 1, 1, 1, 8, 2, 128, 4, 4, 1,
                                               None) == 1
    assert lib.fhip_attention_tq_workspace_bytes(2, 8, 128, 0) == 0
    # split partials: (m, l) and hd floats per (query, head, 1024-position split), 256-aligned
    ml = 4 * 32 * 32 * 2 * 4
    assert lib.fhip_attention_paged_workspace_bytes(4, 32, 128, 2048) == ml + 4 * 32 * 32 * 128 * 4
    assert lib.fhip_attention_paged_workspace_bytes(0, 32, 128, 2048) == 0
    # contiguous-cache attention (ffi.rs:172-184) is a stub: hipErrorNotSupported (801)
    assert lib.fhip_launch_attention(1, 1, 1, 1, 1, 8, 2, 128, 16, 0, None) == 801
    # measurement probes: arguments are checked before any launch
    assert lib.fhip_probe_empty(0, None) == 1
    assert lib.fhip_probe_stream(None, 0, None, 0, 16, None, 1, None) == 1  # moves nothing
    assert lib.fhip_probe_stream(None, 1, None, 0, 16, None, 1, None) == 1  # null input list
    assert lib.fhip_probe_stream(None, 4, None, 0, 16, None, 1, None) == 1  # > 3 inputs
    assert lib.fhip_probe_stream(None, 0, None, 1, 24, None, 1, None) == 1  # not 16-byte units
    # matmul sizes
    assert lib.fhip_launch_matmul(None, None, None, -1, 4, 4, None) == 1
    assert lib.fhip_launch_matmul(None, None, None, 0, 4, 4, None) == 0


def test_batched_attention_wrapper_rejects_length_mismatch():
    """The Python wrapper refuses lengths or block-table rows that do not match q's rows before
    the library reads either host array; matching ones reach the library (which here, with no
    backend, refuses the null handle)."""
    from fracture_amd import BackendError, DeviceTensor, DType, HipBackend, InvalidShape, TensorId

    b = HipBackend.__new__(HipBackend)
    b._L, b._h = _lib.load(), None
    q = DeviceTensor(TensorId(1), (3, 32, 128), DType.FP16)
    t = DeviceTensor(TensorId(2), (128, 128), DType.FP32)
    args = (1, t, t, t, t, 4, 4, 8, q)
    with pytest.raises(InvalidShape, match="2 lengths"):
        b.attention_paged_tq_batched(q, [[0], [1], [2]], [16, 16], *args)
    with pytest.raises(InvalidShape, match="2 block-table rows"):
        b.attention_paged_tq_batched(q, [[0], [1]], [16, 16, 16], *args)
    with pytest.raises(InvalidShape, match="4 block-table rows"):
        b.attention_paged_tq_batched(q, np.zeros((4, 2), np.int32), [16, 16, 16], *args)
    with pytest.raises(BackendError, match="null backend"):
        b.attention_paged_tq_batched(q, [[0], [1], [2]], [16, 16, 16], *args)


def test_kernels_module_requires_device_tensors():
    import torch

    from fracture_amd import kernels as K

    a = torch.zeros(8, dtype=torch.float16)
    with pytest.raises(ValueError):
        K.add(a, a, a)


def _c_params(decl: str) -> int:
    inner = decl[decl.index("(") + 1:decl.rindex(")")].strip()
    return 0 if inner in ("", "void") else inner.count(",") + 1


def test_rust_shim_declarations_match_header():
    """The FFI block of backends/fracture-hip (the Rust crate a Fracture maintainer drops in)
    names only header functions, each with the header's parameter count."""
    import re
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    ffi = (root / "backends/fracture-hip/src/ffi.rs").read_text()
    hdr = (root / "include/fracture_hip.h").read_text()
    decls = re.findall(r"pub fn (fhip_\w+)\(([^;]*?)\)\s*(?:->[^;]*)?;", ffi, re.S)
    assert len(decls) > 40
    for name, args in decls:
        m = re.search(r"\b" + name + r"\s*\(([^;]*?)\)\s*;", hdr, re.S)
        assert m, f"{name} is not declared in the header"
        n_rust = 0 if not args.strip() else args.count(":")
        assert n_rust == _c_params("(" + m.group(1) + ")"), name


# The CUDA backend's raw launchers (backends/fracture-cuda/src/ffi.rs:141-274): name and
# parameter types in order, the types the HIP crate must mirror (c_int dims, device pointers,
# a trailing stream).
REF_LAUNCHERS = {
    "launch_rmsnorm": ["*mut c_void", "*const c_void", "*const c_void", "f32", "c_int", "c_int",
                       "stream"],
    "launch_rope": ["*mut c_void", "*mut c_void", "*const u32", "*const f32", "c_int", "c_int",
                    "c_int", "c_int", "stream"],
    "launch_silu_mul": ["*mut c_void", "*const c_void", "*const c_void", "c_int", "stream"],
    "launch_attention": ["*mut c_void", "*const c_void", "*const c_void", "*const c_void",
                         "c_int", "c_int", "c_int", "c_int", "c_int", "c_int", "stream"],
    "launch_paged_attention": ["*mut c_void", "*const c_void", "*const c_int",
                               "*const *const c_void", "*const *const c_void", "c_int", "c_int",
                               "c_int", "c_int", "c_int", "c_int", "c_int", "stream"],
    "launch_embedding": ["*mut c_void", "*const c_void", "*const u32", "c_int", "c_int", "c_int",
                         "stream"],
    "launch_add": ["*mut c_void", "*const c_void", "*const c_void", "c_int", "stream"],
    "launch_turboquant_compress": ["*const c_void", "*const f32", "*const f32", "*mut c_void",
                                   "*mut c_void", "c_int", "c_int", "c_int", "c_int", "c_int",
                                   "c_int", "stream"],
    "launch_turboquant_decompress": ["*const c_void", "*const c_void", "*const f32",
                                     "*const f32", "*mut c_void", "c_int", "c_int", "c_int",
                                     "c_int", "c_int", "stream"],
    "launch_attention_paged_tq": ["*mut c_void", "*const c_void", "*const c_int"]
    + ["*const *const c_void"] * 4 + ["*const f32"] * 4 + ["c_int"] * 10 + ["stream"],
}


def _rust_fns(src):
    """name -> list of parameter types of each `pub fn` declared in an extern block."""
    import re

    out = {}
    for name, args in re.findall(r"pub fn (\w+)\(([^;{]*?)\)\s*(?:->[^;{]*)?;", src, re.S):
        types = [a.split(":", 1)[1].strip() for a in args.split(",") if ":" in a]
        out[name] = types
    return out


def _rust_src(name):
    from pathlib import Path

    return (Path(__file__).resolve().parents[1] / "backends/fracture-hip/src" / name).read_text()


def test_rust_raw_launchers_match_reference_block():
    """Every launch_* of the reference block exists in the crate's ffi module under its own
    name (a re-export of fhip_launch_*), with the reference's parameter types and a stream."""
    ffi = _rust_src("ffi.rs")
    fns = _rust_fns(ffi)
    for ref_name, ref_types in REF_LAUNCHERS.items():
        assert f"pub use self::fhip_{ref_name} as {ref_name};" in ffi, ref_name
        got = fns["fhip_" + ref_name]
        want = [("hipStream_t" if t == "stream" else t) for t in ref_types]
        assert got == want, (ref_name, got)
    # the stream and status types callers pass and compare (backend.stream(), err == 0)
    assert "pub type hipStream_t = *mut c_void;" in ffi
    assert "pub type hipError_t = c_int;" in ffi


def test_rust_inherent_api_matches_cuda_backend():
    """HipBackend's inherent methods have CudaBackend's signatures (cuda/src/lib.rs:76-161),
    as the bins and tests call them: new(i32), get_ptr(TensorId), stream(),
    precompute_rope_freqs(&mut self, usize, f64)."""
    import re

    be = re.sub(r"\s+", " ", _rust_src("backend.rs"))
    assert "pub fn new(device_id: i32) -> Result<Self>" in be
    assert "pub fn get_ptr(&self, id: TensorId) -> Result<*mut c_void>" in be
    assert "pub fn stream(&self) -> hipStream_t" in be
    assert "pub fn precompute_rope_freqs(&mut self, head_dim: usize, theta: f64) -> Result<()>" in be
    assert "impl Backend for HipBackend" in be and "impl BackendExt for HipBackend" in be


def test_rust_backend_ext_has_defaults_and_overrides():
    """BackendExt declares each additive op with a default body (other backends need no
    change), and HipBackend overrides every one of them."""
    import re

    ext = _rust_src("ext.rs")
    trait = ext[ext.index("pub trait BackendExt: Backend {"):]
    ops = re.findall(r"\n    fn (\w+)\(", trait)
    assert sorted(ops) == sorted(["add_rmsnorm", "softmax_rows", "argmax_rows", "tq_dequantize",
                                  "tq_quantize_pack", "attention_paged_tq_batched"])
    for op in ops:  # a body, not a bare declaration
        sig_end = re.search(r"\n    fn " + op + r"\([^{;]*?\)\s*->\s*Result<[^{;]*?>\s*([{;])", trait, re.S)
        assert sig_end and sig_end.group(1) == "{", op
    be = _rust_src("backend.rs")
    impl = be[be.index("impl BackendExt for HipBackend {"):]
    assert sorted(re.findall(r"\n    fn (\w+)\(", impl)) == sorted(ops)


def test_rust_sources_are_balanced():
    """A cheap syntax screen (no Rust toolchain in the image): brackets balance in every crate
    source once strings, chars and comments are removed."""
    import re

    for name in ("lib.rs", "ffi.rs", "backend.rs", "ext.rs"):
        s = _rust_src(name)
        s = re.sub(r"//[^\n]*", "", s)
        s = re.sub(r'"(?:\\[\s\S]|[^"\\])*"', '""', s)  # a \<newline> continues a string
        s = re.sub(r"'(?:\\.|[^'\\])'", "''", s)
        stack = []
        pairs = {")": "(", "]": "[", "}": "{"}
        for ch in s:
            if ch in "([{":
                stack.append(ch)
            elif ch in ")]}":
                assert stack and stack.pop() == pairs[ch], name
        assert not stack, name
