"""Regenerate tests/golden/tiny_llama_fixture.npz from the reference's committed test data.

Reads (as data, nothing is executed or imported from the reference):
  * tests/reference-fixture/{prompt_0,prompt_1,decode_step_0}/**.bin — PyTorch per-op dumps
    in the reference's tensor format (tests/validation/src/tensor_compare.rs:68-121:
    u32 ndim, u32 shape[ndim], u32 dtype, little-endian data);
  * tests/fixtures/tiny-llama.gguf — the F16 tiny model: every weight tensor (norms, token
    embedding, attention and FFN projections, output head) is extracted (GGUF v3 container:
    header, metadata, tensor infos, aligned data section).

The reference tree lives at /root/reference in the build container; pass another path as
the first argument. The .npz (a few MB at most) is what the tests load.
"""
from __future__ import annotations

import json
import struct
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
OUT = HERE / "tiny_llama_fixture.npz"
CASES = ["prompt_0", "prompt_1", "decode_step_0"]
PER_LAYER = ["input_hidden", "post_attn_norm", "q", "k", "v", "q_rope", "k_rope", "attn_output",
             "post_attn_residual", "post_ffn_norm", "gate", "up", "silu_mul", "ffn_output",
             "output_hidden"]
TOP = ["token_ids", "embeddings", "final_norm", "logits", "greedy_token"]

# dtype codes of the .bin format (tests/validation/src/tensor_compare.rs DType::from_u32)
BIN_DTYPES = {0: np.float32, 1: np.float16, 2: np.int32}


def read_bin(path: Path) -> np.ndarray:
    raw = path.read_bytes()
    ndim = struct.unpack_from("<I", raw, 0)[0]
    shape = struct.unpack_from(f"<{ndim}I", raw, 4)
    code = struct.unpack_from("<I", raw, 4 + 4 * ndim)[0]
    data = raw[8 + 4 * ndim:]
    dt = BIN_DTYPES.get(code)
    n = int(np.prod(shape)) if ndim else 1
    if dt is None or len(data) != n * np.dtype(dt).itemsize:
        # the dtype code is inferred from the byte count when the table above is incomplete
        for cand in (np.float32, np.int32, np.float16):
            if len(data) == n * np.dtype(cand).itemsize:
                dt = cand
                break
    return np.frombuffer(data, dtype=dt).reshape(shape).copy()


def read_gguf_tensors(path: Path, wanted) -> dict:
    raw = path.read_bytes()
    off = 0

    def take(fmt):
        nonlocal off
        v = struct.unpack_from(fmt, raw, off)
        off += struct.calcsize(fmt)
        return v if len(v) > 1 else v[0]

    def gstr():
        n = take("<Q")
        nonlocal off
        s = raw[off:off + n].decode("utf-8")
        off += n
        return s

    scalar = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?",
              10: "<Q", 11: "<q", 12: "<d"}

    def value(t):
        if t in scalar:
            return take(scalar[t])
        if t == 8:
            return gstr()
        if t == 9:
            et = take("<I")
            cnt = take("<Q")
            return [value(et) for _ in range(cnt)]
        raise ValueError(f"GGUF value type {t}")

    assert raw[:4] == b"GGUF", "not a GGUF file"
    off = 4
    version = take("<I")
    n_tensors = take("<Q")
    n_kv = take("<Q")
    meta = {}
    for _ in range(n_kv):
        k = gstr()
        meta[k] = value(take("<I"))
    infos = []
    for _ in range(n_tensors):
        name = gstr()
        nd = take("<I")
        dims = [take("<Q") for _ in range(nd)]
        gt = take("<I")
        toff = take("<Q")
        infos.append((name, dims, gt, toff))
    align = int(meta.get("general.alignment", 32))
    data0 = (off + align - 1) // align * align
    ggml = {0: np.float32, 1: np.float16}
    out = {}
    for name, dims, gt, toff in infos:
        if name not in wanted:
            continue
        dt = ggml[gt]
        n = int(np.prod(dims))
        arr = np.frombuffer(raw, dtype=dt, count=n, offset=data0 + toff)
        out[name] = arr.reshape(list(reversed(dims))).copy()  # ne[0] is innermost
    out["__version__"] = version
    return out


def main(ref_root: Path) -> None:
    fx = ref_root / "tests" / "reference-fixture"
    cfg = json.loads((ref_root / "tests" / "fixtures" / "tiny-llama.config.json").read_text())
    arrays = {}
    for case in CASES:
        d = fx / case
        for t in TOP + (["position_index"] if case.startswith("decode") else []):
            arrays[f"{case}/{t}"] = read_bin(d / f"{t}.bin")
        for layer in range(cfg["num_layers"]):
            for t in PER_LAYER:
                arrays[f"{case}/layer_{layer:02d}/{t}"] = read_bin(d / f"layer_{layer:02d}" / f"{t}.bin")
    names = ["token_embd.weight", "output_norm.weight", "output.weight"]
    for layer in range(cfg["num_layers"]):
        names += [f"blk.{layer}.{t}.weight" for t in
                  ("attn_norm", "ffn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                   "ffn_gate", "ffn_up", "ffn_down")]
    w = read_gguf_tensors(ref_root / "tests" / "fixtures" / "tiny-llama.gguf", set(names))
    for n in names:
        arrays[f"weights/{n}"] = w[n]
    arrays["config"] = np.frombuffer(json.dumps(cfg).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size // 1024} KiB, {len(arrays)} arrays)")


if __name__ == "__main__":
    main(Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference"))
