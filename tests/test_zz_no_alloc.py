"""attention_forward_noalloc: attention_forward with the library's own device workspace (no
allocation by the library or the caller), checked through the C ABI against attention_forward on
the same inputs, bit for bit, on two calls in a row (the second smaller, so it runs on what the
first left in the shared workspace), plus the size limit."""
import ctypes

import numpy as np
import pytest

from conftest import load_package, rand_bf16


def _dev(bits):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).cuda()


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint16)


@pytest.mark.gpu
@pytest.mark.parametrize("first,second", [
    ((32, 8, 8447, 8448), (16, 8, 300, 512)),   # 4B heads at an 8192+ history, then 0.6B heads
    ((16, 8, 4095, 4096), (8, 2, 63, 64)),
])
def test_attention_noalloc_matches_attention_forward(gpu, first, second):
    import torch
    L = gpu.lib()
    D = 128
    scale = float(np.float32(1.0 / np.sqrt(D)))
    for case, (hq, hkv, pos, max_seq) in enumerate((first, second)):
        print(f"[case] noalloc call {case + 1}: {hq}/{hkv} heads, pos {pos}, max_seq {max_seq}",
              flush=True)
        rng = np.random.default_rng(1000 * case + pos)
        q = _dev(rand_bf16(rng, hq * D))
        kc = _dev(rand_bf16(rng, (max_seq, hkv * D)))
        vc = _dev(rand_bf16(rng, (max_seq, hkv * D)))
        d_pos = torch.tensor([pos], dtype=torch.int32, device="cuda")
        att = torch.zeros(gpu.attention_workspace_floats(hq, D, max_seq), dtype=torch.float32,
                          device="cuda")
        want = _dev(np.zeros(hq * D, np.uint16))
        got = _dev(np.full(hq * D, 0x7FC1, np.uint16))
        stream = torch.cuda.current_stream().cuda_stream
        L.attention_forward(want.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                            att.data_ptr(), hq, hkv, D, d_pos.data_ptr(), max_seq, scale, stream)
        L.attention_forward_noalloc(got.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                    hq, hkv, D, d_pos.data_ptr(), max_seq, scale, stream)
        assert L.llm_last_error() is None
        assert np.array_equal(_host(got), _host(want))


def test_attention_noalloc_size_limit():
    """More workspace than the library's array holds is an error before anything is launched
    (host-side: runs in the CPU suite, no GPU call is made)."""
    pkg = load_package()
    L = pkg.lib()
    L.llm_clear_error()
    L.attention_forward_noalloc(0x1000, 0x1000, 0x1000, 0x1000, 32, 8, 128, 0x1000, 10799,
                                0.1, None)
    msg = L.llm_last_error().decode()
    L.llm_clear_error()
    assert "the library's scratch holds 1048576" in msg
