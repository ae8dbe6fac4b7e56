"""The allocation-free decode entry point (ukv_page16_decode_noalloc), through the C ABI.

Its split-K scratch is a device array of the library shared by every call on the GPU, so
the test makes two calls in a row - a ragged 64-sequence batch, then a smaller 4-sequence
fp16 batch that reuses the scratch the first call left behind - and checks each against
ukv_page16_decode with a workspace of its own (bit for bit: the same kernels run) and the
small one against the fp64 oracle as well (|gpu - oracle| <= 2e-3 + 1e-2 |oracle|).
A shape whose scratch exceeds UKV_PAGE16_SCRATCH_BYTES is refused before any launch.
"""
import numpy as np
import pytest

from oracle import oracle
from unifiedkv_amd import _ext, workloads

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20  # UKV_PAGE16_SCRATCH_BYTES in include/ukv.h


def _call(lib, tc, out, workspace=None):
    import torch

    B, Hq, D = (int(x) for x in tc["q"].shape)
    Hkv = int(tc["k_cache"].shape[2])
    mb = int(tc["block_table"].shape[1])
    dt = _ext.UKV_DTYPE_BF16 if tc["q"].dtype == torch.bfloat16 else _ext.UKV_DTYPE_F16
    args = (tc["q"].data_ptr(), tc["k_cache"].data_ptr(), tc["v_cache"].data_ptr(), tc["block_table"].data_ptr(),
            tc["seqlens"].data_ptr(), out.data_ptr(), B, Hq, Hkv, D, Hq // Hkv, mb, int(tc["k_cache"].shape[0]),
            _ext.i64_array(tc["q"].stride()[:2]), _ext.i64_array(tc["k_cache"].stride()[:3]),
            _ext.i64_array(tc["v_cache"].stride()[:3]), float(tc["scale"]), dt)
    stream = torch.cuda.current_stream().cuda_stream
    if workspace is None:
        return lib.ukv_page16_decode_noalloc(*args, stream)
    return lib.ukv_page16_decode(*args, workspace.data_ptr(), workspace.numel(), stream)


def _both(lib, tc):
    import torch

    B, Hq, D = (int(x) for x in tc["q"].shape)
    ws_bytes = int(lib.ukv_page16_workspace_bytes(B, Hq, D, int(tc["block_table"].shape[1])))
    assert 0 < ws_bytes <= SCRATCH_BYTES
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=tc["q"].device)
    ref = torch.empty_like(tc["q"])
    assert _call(lib, tc, ref, ws) == _ext.UKV_OK
    got = torch.full_like(tc["q"], float("nan"))
    assert _call(lib, tc, got) == _ext.UKV_OK
    torch.cuda.synchronize()
    return got, ref


def test_noalloc_matches_workspace_entry_point_twice(cuda):
    import torch

    lib = _ext.load()
    print("[no_alloc] call 1: ragged B=64 bf16, seed 7", flush=True)
    big = workloads.torch_decode_case(workloads.layout_ragged(np.random.default_rng(7)), 7, device=cuda)
    got, ref = _both(lib, big)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), "call 1 differs from ukv_page16_decode"
    del big

    print("[no_alloc] call 2: config-1 tiny B=4 fp16, seed 11", flush=True)
    case = workloads.numpy_case("tiny", 11)
    small = workloads.to_torch(case, cuda)
    got, ref = _both(lib, small)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), "call 2 differs from ukv_page16_decode"
    f = lambda a: oracle.bits_to_f32(a, oracle.DT_F16)
    exp = oracle.page16_decode_dense(f(case["q"]), f(case["k_cache"]), f(case["v_cache"]), case["block_table"],
                                     case["seqlens"], softmax_scale=case["scale"], n_rep=case["n_rep"])
    ok, max_err, excess = oracle.allclose_report(got.float().cpu().numpy(), exp, 2e-3, 1e-2)
    assert ok, f"call 2 vs oracle: max_abs_err={max_err:.3e} worst_excess={excess:.3e}"


def test_noalloc_refuses_shapes_beyond_its_scratch(cuda):
    lib = _ext.load()
    B, Hq, D, mb = 5000, 64, 256, 4
    assert int(lib.ukv_page16_workspace_bytes(B, Hq, D, mb)) > SCRATCH_BYTES
    z = _ext.i64_array([0, 0, 0])
    rc = lib.ukv_page16_decode_noalloc(None, None, None, None, None, None, B, Hq, 8, D, Hq // 8, mb, 1, z, z, z,
                                       1.0, _ext.UKV_DTYPE_BF16, None)
    assert rc == _ext.UKV_ERR_WORKSPACE
