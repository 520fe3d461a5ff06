"""Tile intersection, radix sort and tile offsets on the GPU: bit-exact
against the host oracle (reference test: tests/test_basic.py:698-736)."""

import math

import numpy as np
import pytest
import torch

from oracle import exact
from tests._util import DEV

pytestmark = pytest.mark.gpu


def _compare(got, want):
    for name, g, w in zip(("tiles_per_gauss", "isect_ids", "flatten_ids"), got, want):
        np.testing.assert_array_equal(g.cpu().numpy(), w, err_msg=name)


@pytest.mark.parametrize("batch_dims", [(), (2,), (1, 2)])
def test_isect_box_reference_inputs(batch_dims):
    """The reference's own test inputs: C=3, N=1000, 40x60 image, random radii."""
    from gsplat_amd.cuda._wrapper import isect_offset_encode, isect_tiles
    rng = np.random.default_rng(42)
    C, N, W, H, ts = 3, 1000, 40, 60, 16
    means2d = (rng.standard_normal((C, N, 2)) * W).astype(np.float32)
    radii = rng.integers(0, W, (C, N, 2)).astype(np.int32)
    depths = rng.random((C, N)).astype(np.float32)
    if batch_dims:
        reps = int(np.prod(batch_dims))
        means2d = np.broadcast_to(means2d, batch_dims + means2d.shape).copy()
        radii = np.broadcast_to(radii, batch_dims + radii.shape).copy()
        depths = np.broadcast_to(depths, batch_dims + depths.shape).copy()
    I = means2d.size // (N * 2)
    tw, th = math.ceil(W / ts), math.ceil(H / ts)
    got = isect_tiles(torch.from_numpy(means2d).to(DEV), torch.from_numpy(radii).to(DEV),
                      torch.from_numpy(depths).to(DEV), ts, tw, th)
    want = exact.isect_tiles_box_python(means2d, radii, depths, ts, tw, th)
    _compare(got, want)
    offs = isect_offset_encode(got[1], I, tw, th)
    np.testing.assert_array_equal(offs.cpu().numpy(),
                                  exact.isect_offset_encode(want[1], I, tw, th))


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("accutile", [False, True])
def test_isect_projected_scene(packed, accutile):
    from gsplat_amd.cuda._wrapper import isect_offset_encode, isect_tiles
    from tests._util import small_scene
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=5, N=20000, C=3, W=320, H=200)
    ex = exact.projection_fwd(means.numpy(), None, quats.numpy(), scales.numpy(),
                              opac.numpy(), vm.numpy(), K.numpy(), W, H)
    C, N = 3, means.shape[0]
    ts = 16
    tw, th = math.ceil(W / ts), math.ceil(H / ts)
    ops = np.broadcast_to(opac.numpy()[None], (C, N)).copy()
    if packed:
        rows = np.nonzero(ex["valid"].reshape(-1))[0]
        m2 = ex["means2d"].reshape(-1, 2)[rows]
        rad = ex["radii"].reshape(-1, 2)[rows]
        dep = ex["depths"].reshape(-1)[rows]
        con = ex["conics"].reshape(-1, 3)[rows]
        op = ops.reshape(-1)[rows]
        iid = (rows // N).astype(np.int64)
        gid = (rows % N).astype(np.int64)
        kw = dict(conics=con, opacities=op) if accutile else {}
        want = exact.isect_tiles(m2, rad, dep, ts, tw, th, packed=True, n_images=C,
                                 image_ids=iid, **kw)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
        got = isect_tiles(t(m2), t(rad), t(dep), ts, tw, th, packed=True, n_images=C,
                          image_ids=t(iid), gaussian_ids=t(gid),
                          conics=t(con) if accutile else None,
                          opacities=t(op) if accutile else None)
    else:
        kw = dict(conics=ex["conics"], opacities=ops) if accutile else {}
        want = exact.isect_tiles(ex["means2d"], ex["radii"], ex["depths"], ts, tw, th, **kw)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
        got = isect_tiles(t(ex["means2d"]), t(ex["radii"]), t(ex["depths"]), ts, tw, th,
                          conics=t(ex["conics"]) if accutile else None,
                          opacities=t(ops) if accutile else None)
    assert want[1].shape[0] > 1000
    _compare(got, want)
    offs = isect_offset_encode(got[1], C, tw, th)
    np.testing.assert_array_equal(offs.cpu().numpy(), exact.isect_offset_encode(want[1], C, tw, th))


@pytest.mark.parametrize("W,H,C", [(64, 48, 2), (1024, 1024, 3)])
def test_isect_sorted_with_depth_ties(W, H, C):
    """Quantised depths make many (image, tile, depth) keys equal: the sorted
    order must still be by (key, row).  The 1024x1024 case has a 13-bit tile
    key (4096 tiles) and a 2-bit image id, so the tile stage takes two
    radix passes; the small case one."""
    from gsplat_amd.cuda._wrapper import isect_tiles
    rng = np.random.default_rng(W)
    N, ts = 6000, 16
    tw, th = math.ceil(W / ts), math.ceil(H / ts)
    means2d = np.stack([rng.uniform(-20, W + 20, (C, N)),
                        rng.uniform(-20, H + 20, (C, N))], -1).astype(np.float32)
    radii = rng.integers(0, 40, (C, N, 2)).astype(np.int32)
    depths = np.round(rng.uniform(1, 3, (C, N)) * 4).astype(np.float32) / 4
    want = exact.isect_tiles(means2d, radii, depths, ts, tw, th)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    got = isect_tiles(t(means2d), t(radii), t(depths), ts, tw, th)
    assert want[1].shape[0] > 5000
    _compare(got, want)


def test_isect_unsorted_emission_order():
    from gsplat_amd.cuda._wrapper import isect_tiles
    from tests._util import small_scene
    means, quats, scales, opac, vm, K, W, H = small_scene(seed=6, N=3000, C=1)
    ex = exact.projection_fwd(means.numpy(), None, quats.numpy(), scales.numpy(),
                              opac.numpy(), vm.numpy(), K.numpy(), W, H)
    want = exact.isect_tiles(ex["means2d"], ex["radii"], ex["depths"], 16, 10, 8, sort=False,
                             conics=ex["conics"], opacities=opac.numpy()[None])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    got = isect_tiles(t(ex["means2d"]), t(ex["radii"]), t(ex["depths"]), 16, 10, 8,
                      sort=False, conics=t(ex["conics"]), opacities=t(opac.numpy()[None]))
    _compare(got, want)


# 2_100_001 exceeds the short-tile limit (2^21 keys) of the sort
@pytest.mark.parametrize("n", [1, 100, 4096, 4097, 300_001, 2_100_001])
@pytest.mark.parametrize("bits", [8, 13, 37, 45, 47, 64])
def test_radix_sort_pairs_stable(n, bits):
    from gsplat_amd import _lib
    rng = np.random.default_rng(n + bits)
    hi = np.uint64((1 << bits) - 1) if bits < 64 else np.uint64(0xFFFFFFFFFFFFFFFF)
    keys = rng.integers(0, 2 ** 63, n, dtype=np.int64).astype(np.uint64) * np.uint64(2) \
        + rng.integers(0, 2, n).astype(np.uint64)
    keys &= hi
    # many duplicates to exercise stability
    keys[rng.random(n) < 0.3] = keys[0]
    vals = np.arange(n, dtype=np.uint32)
    kd = torch.from_numpy(keys.view(np.int64)).to(DEV)
    vd = torch.from_numpy(vals.view(np.int32)).to(DEV)
    ko, vo = torch.empty_like(kd), torch.empty_like(vd)
    ws = torch.empty(_lib.query("gsplat_sort_pairs_workspace_size", n), dtype=torch.uint8,
                     device=DEV)
    _lib.call("gsplat_sort_pairs_u64_u32", n, bits, kd.data_ptr(), vd.data_ptr(),
              ko.data_ptr(), vo.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream())
    order = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(ko.cpu().numpy().view(np.uint64), keys[order])
    np.testing.assert_array_equal(vo.cpu().numpy().view(np.uint32), vals[order])


def test_offsets_empty_and_zero_isects():
    from gsplat_amd.cuda._wrapper import isect_offset_encode
    offs = isect_offset_encode(torch.empty(0, dtype=torch.int64, device=DEV), 2, 5, 4)
    assert offs.shape == (2, 4, 5) and int(offs.abs().sum()) == 0


@pytest.mark.parametrize("N", [200, 700, 1400, 2800, 11000])
def test_tile_first_sort_every_segment_size(N):
    """The tile-first sorted intersection sorts each tile's rows on their
    depth bits in LDS (2,560 rows where tiles average up to 1,500 rows,
    else 4,096) and through global scratch above that.  Rows with large
    radii put about N rows into each of the 12 tiles of every image: N up to
    1,400 takes the 1-, 5- and 10-key paths of the smaller LDS, 2,800 the
    16-key path of the larger one and 11,000 its global scratch.
    Depths are quantised (many ties, which must stay in row order) and half
    of them negative (their zero-extended bits order after every positive
    depth, IntersectTile.cu:190-192).  The offsets come from the same call
    and must equal the offset encoding of the oracle's ids."""
    from gsplat_amd.cuda import _ops
    rng = np.random.default_rng(N)
    C, ts, W, H = 2, 16, 64, 48
    tw, th = math.ceil(W / ts), math.ceil(H / ts)
    means2d = np.stack([rng.uniform(0, W, (C, N)), rng.uniform(0, H, (C, N))],
                       -1).astype(np.float32)
    radii = rng.integers(40, 90, (C, N, 2)).astype(np.int32)
    radii[:, ::97] = 0  # a few rows with no tile
    depths = (np.round(rng.uniform(-3, 3, (C, N)) * 8) / 8).astype(np.float32)
    want = exact.isect_tiles(means2d, radii, depths, ts, tw, th)
    per_tile = np.bincount(want[1] >> 32, minlength=C * tw * th)
    lo, hi = {200: (1, 256), 700: (513, 1280), 1400: (1281, 2560), 2800: (2561, 4096),
              11000: (4097, None)}[N]
    assert per_tile.max() >= lo and (hi is None or per_tile.max() <= hi), per_tile.max()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    tpg = torch.empty((C, N), dtype=torch.int32, device=DEV)
    state = _ops.isect_prepare_sorted(t(means2d), t(radii), t(depths), None, None,
                                      None, N, C, ts, tw, th, tpg)
    got = _ops.isect_emit_sorted(state)
    _compare(got[:3], want)
    np.testing.assert_array_equal(got[3].cpu().numpy().reshape(-1),
                                  exact.isect_offset_encode(want[1], C, tw, th).reshape(-1))
    # the queued (device-count) form with a capacity above the count
    state = _ops.isect_prepare_sorted(t(means2d), t(radii), t(depths), None, None,
                                      None, N, C, ts, tw, th, tpg)
    _ops.isect_emit_sorted_queue(state, want[1].shape[0] + 1000)
    got = _ops.isect_emit_sorted(state)
    _compare(got[:3], want)
    np.testing.assert_array_equal(got[3].cpu().numpy().reshape(-1),
                                  exact.isect_offset_encode(want[1], C, tw, th).reshape(-1))


@pytest.mark.parametrize("counts", [
    # mean 1,008 rows a tile: the 2,560-row LDS (1, 2, 5 or 10 keys a
    # thread, then global scratch)
    (200, 400, 700, 1400, 2800, 6000, 100, 100, 100, 100, 100, 100),
    # mean 2,950: the 4,096-row LDS (2, 4, 8 or 16 keys a thread, then global
    # scratch)
    (200, 700, 1500, 3000, 6000, 4000, 4000, 4000, 4000, 4000, 2000, 2000),
])
def test_tile_depth_sort_every_path(counts):
    """Rows of radius 2 px at tile centres, so every row lands in one tile and
    each tile of the 3 x 4 image holds the given number of rows.  The mean
    tile depth picks the LDS capacity of the per-tile depth sort, and the
    tiles' sizes take every path of that capacity.  Depths are quantised
    (ties stay in row order) and a third of them negative (zero-extended
    bits order after every positive depth, IntersectTile.cu:190-192).  Ids,
    rows and offsets must equal the oracle's."""
    from gsplat_amd.cuda import _ops
    rng = np.random.default_rng(sum(counts))
    C, ts, tw, th = 1, 16, 4, 3
    W, H = tw * ts, th * ts
    tile_of = np.repeat(np.arange(tw * th), counts)
    rng.shuffle(tile_of)
    N = tile_of.size
    cx = (tile_of % tw) * ts + 8 + rng.uniform(-4, 4, N)
    cy = (tile_of // tw) * ts + 8 + rng.uniform(-4, 4, N)
    means2d = np.stack([cx, cy], -1)[None].astype(np.float32)
    radii = np.full((C, N, 2), 2, dtype=np.int32)
    depths = (np.round(rng.uniform(-2, 4, (C, N)) * 16) / 16).astype(np.float32)
    want = exact.isect_tiles(means2d, radii, depths, ts, tw, th)
    np.testing.assert_array_equal(np.bincount(want[1] >> 32, minlength=tw * th), counts)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    tpg = torch.empty((C, N), dtype=torch.int32, device=DEV)
    state = _ops.isect_prepare_sorted(t(means2d), t(radii), t(depths), None, None,
                                      None, N, C, ts, tw, th, tpg)
    got = _ops.isect_emit_sorted(state)
    _compare(got[:3], want)
    np.testing.assert_array_equal(got[3].cpu().numpy().reshape(-1),
                                  exact.isect_offset_encode(want[1], C, tw, th).reshape(-1))


@pytest.mark.parametrize("group,negative", [(12, False), (12, True), (80, False)])
def test_tile_depth_sort_clustered_depths(group, negative):
    """Depths in clusters of about `group` rows per tile, each cluster a few
    dozen float ulps wide in random row order, clusters 0.01 apart and a few
    far depths (12.0, or -1.0 whose bits order last) widening every tile's
    range.  The per-tile sort ranks the top bits of the range by radix passes
    and orders the rows that tie on those bits afterwards: clusters of 12 are
    such runs with their low bits out of order, clusters of 80 exceed the
    run limit and take the full-key passes.  The ids must equal the oracle's
    stable sort (IntersectTile.cu:496-505)."""
    from gsplat_amd.cuda import _ops
    N = 1500
    rng = np.random.default_rng(group + int(negative))
    C, ts, W, H = 1, 16, 64, 48
    tw, th = math.ceil(W / ts), math.ceil(H / ts)
    means2d = np.stack([rng.uniform(0, W, (C, N)), rng.uniform(0, H, (C, N))],
                       -1).astype(np.float32)
    radii = rng.integers(40, 90, (C, N, 2)).astype(np.int32)
    g = rng.integers(0, max(N // group, 1), (C, N))
    depths = (2.0 + 0.01 * g + rng.uniform(0, 2e-5, (C, N))).astype(np.float32)
    depths[:, ::150] = -1.0 if negative else 12.0
    want = exact.isect_tiles(means2d, radii, depths, ts, tw, th)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    tpg = torch.empty((C, N), dtype=torch.int32, device=DEV)
    state = _ops.isect_prepare_sorted(t(means2d), t(radii), t(depths), None, None,
                                      None, N, C, ts, tw, th, tpg)
    got = _ops.isect_emit_sorted(state)
    _compare(got[:3], want)


def _depth_first(means2d, radii, depths, C, N, ts, tw, th, capacity=None):
    """The depth-first two-stage form through the C ABI directly
    (gsplat_isect_prepare, then gsplat_isect_emit_sorted or, with a
    capacity, gsplat_isect_emit_sorted_dev)."""
    from gsplat_amd.cuda._ops import _stream, call, ptr, query
    n = C * N
    tpg = torch.empty(n, dtype=torch.int32, device=DEV)
    order = torch.empty(n, dtype=torch.int32, device=DEV)
    starts = torch.empty(n + 1, dtype=torch.int64, device=DEV)
    recs = torch.empty(n, 8, dtype=torch.float32, device=DEV)
    total = torch.empty(1, dtype=torch.int64, device=DEV)
    ws = torch.empty(query("gsplat_isect_prepare_workspace_size", n), dtype=torch.uint8,
                     device=DEV)
    st = _stream(means2d)
    call("gsplat_isect_prepare", n, N, None, ptr(means2d), ptr(radii), ptr(depths),
         None, None, ts, tw, th, ptr(ws), ws.numel(), ptr(tpg), ptr(order), ptr(starts),
         ptr(recs), ptr(total), st)
    n_isects = int(total.item())
    size = n_isects if capacity is None else capacity
    ids = torch.empty(size, dtype=torch.int64, device=DEV)
    flat = torch.empty(size, dtype=torch.int32, device=DEV)
    ews = torch.empty(query("gsplat_isect_emit_sorted_workspace_size", size),
                      dtype=torch.uint8, device=DEV)
    name = "gsplat_isect_emit_sorted" if capacity is None else "gsplat_isect_emit_sorted_dev"
    call(name, n, N, C, None, ptr(means2d), ptr(radii), ptr(depths), None, None, ts, tw,
         th, ptr(order), ptr(starts), ptr(recs), size, ptr(ews), ews.numel(), ptr(ids),
         ptr(flat), st)
    return tpg.reshape(C, N), ids[:n_isects], flat[:n_isects]


def test_depth_first_form_matches_oracle():
    """The depth-first form (rows sorted by depth over the whole array, then
    the tile sort) stays exported: bit-exact against the oracle, with
    quantised depths (ties) half of them negative, exact and queued."""
    rng = np.random.default_rng(11)
    C, N, ts, W, H = 2, 5000, 16, 200, 120
    tw, th = math.ceil(W / ts), math.ceil(H / ts)
    means2d = np.stack([rng.uniform(-20, W + 20, (C, N)),
                        rng.uniform(-20, H + 20, (C, N))], -1).astype(np.float32)
    radii = rng.integers(0, 30, (C, N, 2)).astype(np.int32)
    depths = (np.round(rng.uniform(-3, 3, (C, N)) * 8) / 8).astype(np.float32)
    want = exact.isect_tiles(means2d, radii, depths, ts, tw, th)
    assert want[1].shape[0] > 20000
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    _compare(_depth_first(t(means2d), t(radii), t(depths), C, N, ts, tw, th), want)
    _compare(_depth_first(t(means2d), t(radii), t(depths), C, N, ts, tw, th,
                          capacity=want[1].shape[0] + 777), want)
