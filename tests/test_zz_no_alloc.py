"""The allocation-free packed projection (gsplat_projection_packed_fwd_noalloc)
through the C ABI: same outputs, bit for bit, as the workspace entry point
gsplat_projection_packed_fwd, on two calls in a row (the second on a smaller
input, so stale scratch from the first would show), and a clear error above
its row limit."""

import pytest
import torch

from gsplat_amd import _lib
from tests._util import DEV, small_scene

pytestmark = pytest.mark.gpu


def _outputs(B, C, N, dev, comp):
    cap = B * C * N
    return {
        "indptr": torch.full((B * C + 1,), -7, dtype=torch.int32, device=dev),
        "batch_ids": torch.full((cap,), -7, dtype=torch.int64, device=dev),
        "camera_ids": torch.full((cap,), -7, dtype=torch.int64, device=dev),
        "gaussian_ids": torch.full((cap,), -7, dtype=torch.int64, device=dev),
        "radii": torch.full((cap, 2), -7, dtype=torch.int32, device=dev),
        "means2d": torch.full((cap, 2), -7.0, device=dev),
        "depths": torch.full((cap,), -7.0, device=dev),
        "conics": torch.full((cap, 3), -7.0, device=dev),
        "comps": torch.full((cap,), -7.0, device=dev) if comp else None,
        "nnz": torch.full((1,), -7, dtype=torch.int64, device=dev),
        "row_of": torch.full((cap,), -7, dtype=torch.int32, device=dev),
        "row_op": torch.full((cap,), -7.0, device=dev),
    }


def _call(noalloc, ins, W, H, comp):
    means, quats, scales, opac, vm, K = ins
    B, C, N = 1, vm.shape[0], means.shape[0]
    o = _outputs(B, C, N, means.device, comp)
    common = [B, C, N, _lib.ptr(means), None, _lib.ptr(quats), _lib.ptr(scales),
              _lib.ptr(opac), _lib.ptr(vm), _lib.ptr(K), W, H, 0.3, 0.01, 1e10, 0.0, 0]
    outs = [_lib.ptr(o[k]) for k in ("indptr", "batch_ids", "camera_ids", "gaussian_ids",
                                     "radii", "means2d", "depths", "conics", "comps",
                                     "nnz", "row_of", "row_op")]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        _lib.call("gsplat_projection_packed_fwd_noalloc", *common, *outs, stream)
    else:
        ws = torch.empty(_lib.query("gsplat_projection_packed_workspace_size", B, C, N),
                         dtype=torch.uint8, device=means.device)
        _lib.call("gsplat_projection_packed_fwd", *common, _lib.ptr(ws), ws.numel(),
                  *outs, stream)
    torch.cuda.synchronize()
    return o


@pytest.mark.parametrize("comp", [False, True])
def test_noalloc_packed_fwd_matches_workspace_entry(comp):
    for seed, N, C in ((0, 300_000, 3), (1, 20_000, 2)):
        means, quats, scales, opac, vm, K, W, H = small_scene(seed=seed, N=N, C=C)
        ins = [t.to(DEV).contiguous() for t in (means, quats, scales, opac, vm, K)]
        ref = _call(False, ins, W, H, comp)
        got = _call(True, ins, W, H, comp)
        nnz = int(ref["nnz"].item())
        print(f"[noalloc] seed {seed}: N={N} C={C} -> {nnz} rows", flush=True)
        assert nnz > 1000 and int(got["nnz"].item()) == nnz
        for k in ref:
            if ref[k] is None:
                continue
            a, b = got[k], ref[k]
            if k not in ("indptr", "nnz", "row_of"):
                a, b = a[:nnz], b[:nnz]
            assert torch.equal(a, b), k


def test_noalloc_rejects_inputs_above_its_limit():
    limit = _lib.query("gsplat_projection_packed_fwd_noalloc_max_rows")
    assert limit == 65536 * 4096
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=2, N=64, C=1)
    ins = [t.to(DEV).contiguous() for t in (means, quats, scales, opac, vm, K)]
    d = _outputs(1, 1, 64, DEV, False)
    N = limit + 1  # sizes only: rejected before any launch
    with pytest.raises(RuntimeError, match="exceed the static scratch"):
        _lib.call("gsplat_projection_packed_fwd_noalloc", 1, 1, N, _lib.ptr(ins[0]), None,
                  _lib.ptr(ins[1]), _lib.ptr(ins[2]), _lib.ptr(ins[3]), _lib.ptr(ins[4]),
                  _lib.ptr(ins[5]), W, H, 0.3, 0.01, 1e10, 0.0, 0,
                  *[_lib.ptr(d[k]) for k in ("indptr", "batch_ids", "camera_ids",
                                             "gaussian_ids", "radii", "means2d", "depths",
                                             "conics", "comps", "nnz", "row_of", "row_op")],
                  torch.cuda.current_stream().cuda_stream)
