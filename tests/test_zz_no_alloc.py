"""xfh_triangle_multiplication_noalloc (the entry point that allocates nothing; its scratch
is a device array the library holds) against xfh_triangle_multiplication with a caller
workspace, through the C ABI: bit-identical results on consecutive calls, the second one
smaller than the first (so the scratch still holds the first call's larger contents), on
the bf16 fast path and the fp32 general path; too large a problem is refused."""

import pytest
import torch

from oracle import restatement as R
from tests.test_gpu_ops import announce
from xfold_cpu_amd.fastnn import native_hip as nh
from xfold_cpu_amd.synthetic import init_module_

pytestmark = pytest.mark.gpu


def trimul_args(module, pair, mask, dtype, out, accumulate):
    """The argument list of both entry points up to (and without) the workspace."""
    names = ("projection", "gate", "output_projection", "gating_linear")
    w = {name: getattr(module, name).weight.detach().to(dtype).contiguous() for name in names}
    ln_in, ln_c = module.left_norm_input, module.center_norm
    keep = [w, ln_in.weight, ln_in.bias, ln_c.weight, ln_c.bias]
    n, c = pair.shape[0], pair.shape[2]
    args = [nh.ptr(pair), nh.dtype_code(pair.dtype), nh.ptr(mask), nh.F32, n, c,
            int(module.equation == "cik,cjk->cij"), nh.ptr(ln_in.weight), nh.ptr(ln_in.bias),
            float(ln_in.eps), nh.ptr(w["projection"]), nh.ptr(w["gate"]), nh.ptr(ln_c.weight),
            nh.ptr(ln_c.bias), float(ln_c.eps), nh.ptr(w["output_projection"]),
            nh.ptr(w["gating_linear"]), nh.dtype_code(dtype), nh.ptr(out), nh.dtype_code(out.dtype),
            int(accumulate)]
    return args, keep


def run_pair(device, n, outgoing, dtype, seed):
    module = init_module_(R.TriangleMultiplication(128, _outgoing=outgoing).eval(), seed=seed,
                          ln_jitter=True).to(device)
    g = torch.Generator().manual_seed(seed)
    pair = torch.randn(n, n, 128, generator=g).to(dtype).to(device)
    seq = torch.ones(n)
    seq[-3:] = 0
    mask = (seq[:, None] * seq[None, :]).to(device)
    stream = nh.stream_of(torch.device(device))
    results = []
    for accumulate in (False, True):
        base = torch.randn(n, n, 128, generator=g).to(dtype).to(device)
        out_ws, out_na = base.clone(), base.clone()
        args, keep = trimul_args(module, pair, mask, dtype, out_ws, accumulate)
        lib = nh.load_library()
        ws = nh.workspace(lib.xfh_triangle_multiplication_workspace_size(n, 128, nh.dtype_code(dtype)),
                          pair.device)
        nh.call("xfh_triangle_multiplication", *args, nh.ptr(ws), ws.numel(), stream)
        args, keep2 = trimul_args(module, pair, mask, dtype, out_na, accumulate)
        nh.call("xfh_triangle_multiplication_noalloc", *args, stream)
        torch.cuda.synchronize()
        results.append((out_ws.cpu(), out_na.cpu()))
    return results


@pytest.mark.parametrize("dtype,sizes", [(torch.bfloat16, (300, 77)), (torch.float32, (100, 41))])
@pytest.mark.parametrize("outgoing", [True, False])
def test_noalloc_matches_workspace_entry_point(device, dtype, sizes, outgoing):
    for i, n in enumerate(sizes):
        announce("trimul noalloc", dtype, n, outgoing, "call", i + 1)
        for out_ws, out_na in run_pair(device, n, outgoing, dtype, seed=n + i):
            assert torch.isfinite(out_ws.float()).all()
            assert torch.equal(out_ws, out_na), f"n={n}: max diff {(out_ws.float() - out_na.float()).abs().max()}"


def test_noalloc_rejects_problems_beyond_its_scratch(device):
    """n = 600 in bf16 needs ~280 MB of scratch: refused before any launch."""
    module = R.TriangleMultiplication(128).eval().to(device)
    pair = torch.zeros(600, 600, 128, dtype=torch.bfloat16, device=device)
    out = torch.empty_like(pair)
    args, keep = trimul_args(module, pair, None, torch.bfloat16, out, False)
    args[3] = nh.BOOL
    with pytest.raises(ValueError, match="scratch"):
        nh.call("xfh_triangle_multiplication_noalloc", *args, nh.stream_of(pair.device))
