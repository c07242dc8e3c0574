"""fhip_launch_attention_paged_tq_noalloc through the C ABI: the same bytes as
fhip_launch_attention_paged_tq (which takes its partials from a stream-ordered allocation) on
two calls in a row, the second with a smaller input, and the size limit of its static
scratch refused on the host."""
import numpy as np
import pytest
import torch

from fracture_amd import kernels as K
from test_gpu_attention_long import _ptr_table, gpu_pool

pytestmark = pytest.mark.gpu

HIP_ERROR_OUT_OF_MEMORY = 2


def _call(fn, pool, dev, q, kv_len, kbits, vbits, kvh):
    T, qh, hd = q.shape
    ptrs = _ptr_table(pool, dev)
    table = torch.from_numpy(pool["table"][0]).to(dev)
    d = pool["d"]
    out = torch.full_like(q, float("nan"))
    code = fn(out.data_ptr(), q.data_ptr(), table.data_ptr(), ptrs[0].data_ptr(),
              ptrs[1].data_ptr(), ptrs[2].data_ptr(), ptrs[3].data_ptr(), d["krot"].data_ptr(),
              d["vrot"].data_ptr(), d["kc"].data_ptr(), d["vc"].data_ptr(), T, qh, kvh, hd,
              kv_len, kv_len - T, kbits, vbits, K.packed_dim(hd, kbits), K.packed_dim(hd, vbits),
              torch.cuda.current_stream().cuda_stream)
    assert code == 0, code
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_noalloc_matches_allocating_entry(dev):
    lib = K._L()
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    # call 1: causal prefill, 6 queries at 5000 positions, K4/V4 (the MFMA kernel)
    # call 2: one decode query at 1500 positions, K4/V2 (the VALU kernel): a smaller input
    for T, kv_len, qh, kvh, kbits, vbits in ((6, 5000, 32, 8, 4, 4), (1, 1500, 8, 2, 4, 2)):
        print(f"noalloc case T={T} kv_len={kv_len} K{kbits}/V{vbits}", flush=True)
        pool = gpu_pool(dev, kv_len, [kv_len], kvh, 128, kbits, vbits, extra_pages=2)
        q = torch.randn((T, qh, 128), generator=g, device=dev).to(torch.float16)
        want = _call(lib.fhip_launch_attention_paged_tq, pool, dev, q, kv_len, kbits, vbits, kvh)
        got = _call(lib.fhip_launch_attention_paged_tq_noalloc, pool, dev, q, kv_len, kbits,
                    vbits, kvh)
        assert not np.isnan(want.astype(np.float32)).any()
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), \
            f"T={T} kv_len={kv_len}: no-alloc output differs"


def test_noalloc_refuses_oversized_partials():
    """64 queries of 32 heads at 1,048,576 positions need ~1.1 GB of partials: refused before
    anything is launched (only sizes are looked at)."""
    lib = K._L()
    need = lib.fhip_attention_tq_workspace_bytes(64, 32, 128, 65536)
    assert need > 32 << 20
    code = lib.fhip_launch_attention_paged_tq_noalloc(
        1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 64, 32, 8, 128, 1 << 20, (1 << 20) - 64, 4, 4, 64, 64,
        None)
    assert code == HIP_ERROR_OUT_OF_MEMORY
