"""Pins the oracle's geometric and optimizer conventions (CPU only).

The GPU kernels equal the oracle bit for bit, so a convention that kernel and
oracle share wrongly would pass every parity test.  Each check here compares
the oracle with a closed form fixed by the reference's documented conventions
and is shown to reject a plausible slip planted in a copy of the oracle:
  - quaternion (w, x, y, z) -> rotation matrix
    (docs/source/conventions/data_conventions.rst:10-19,
    gsplat/cuda/_math.py:649-669);
  - the view matrix as the world -> camera transform, OpenCV axes
    (data_conventions.rst:21-24; ProjectionEWA3DGSFused.cu:76-92);
  - the camera centre -R^T t and the view direction mean - centre used by SH
    (gsplat/rendering.py:216-253);
  - Adam's moment decay (gsplat/cuda/csrc/AdamCUDA.cu:56-68).
"""

import ctypes
import inspect
import math
import subprocess
import textwrap

import numpy as np
import pytest
import torch
from scipy.spatial.transform import Rotation

from oracle import exact, torch_ref


# --------------------------------------------------------------------------
# planting slips in copies of the oracle
# --------------------------------------------------------------------------
def _mutated_c_oracle(tmp_path, old, new):
    """The C oracle rebuilt with ``old`` replaced by ``new`` (exactly once)."""
    src = (exact._HERE / "exact_ref.c").read_text()
    assert src.count(old) == 1, ("pattern not found once in the oracle", old)
    path = tmp_path / "mutated.c"
    path.write_text(src.replace(old, new))
    so = tmp_path / "libmutated.so"
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off",
                    "-o", str(so), str(path), "-lm"], check=True)
    return ctypes.CDLL(str(so))


def _mutated_py(module, name, old, new):
    """A copy of ``module.name`` compiled from its source with ``old``
    replaced by ``new`` (exactly once), resolving globals in ``module``."""
    src = textwrap.dedent(inspect.getsource(getattr(module, name)))
    assert src.count(old) == 1, ("pattern not found once in", name, old)
    ns = dict(vars(module))
    exec(compile(src.replace(old, new), f"<mutated {name}>", "exec"), ns)
    return ns[name]


class _using_c_oracle:
    """Context manager: route ``exact`` through another build of the C oracle."""

    def __init__(self, lib):
        self.lib = lib

    def __enter__(self):
        self.saved = exact._lib
        if self.lib is not None:
            exact._lib = self.lib

    def __exit__(self, *exc):
        exact._lib = self.saved


# --------------------------------------------------------------------------
# cameras built from the documented convention, independently of the package
# --------------------------------------------------------------------------
def _look_at(p, target=(0.0, 0.0, 0.0), up=(0.0, -1.0, 0.0)):
    """World -> camera matrix of an OpenCV camera (x right, y down, z forward)
    at p looking at target: rows of R are the camera axes in world
    coordinates, t = -R p.  Returns (viewmat 4x4 float64, R)."""
    p = np.asarray(p, np.float64)
    z = np.asarray(target, np.float64) - p
    z /= np.linalg.norm(z)
    x = np.cross(z, np.asarray(up, np.float64))
    x /= np.linalg.norm(x)
    y = np.cross(z, x)
    R = np.stack([x, y, z])
    vm = np.eye(4)
    vm[:3, :3] = R
    vm[:3, 3] = -R @ p
    return vm, R


_CAMERA_POSITIONS = [(3.0, -1.0, 4.0), (-5.0, 2.0, 1.0), (0.5, -4.0, -3.0),
                     (-2.0, -2.0, -6.0)]


def _wxyz(rot: Rotation) -> np.ndarray:
    x, y, z, w = rot.as_quat()
    return np.array([w, x, y, z])


# --------------------------------------------------------------------------
# Quaternion -> rotation
# --------------------------------------------------------------------------
def _quat_rot_error_torch(fn):
    """Largest deviation of fn (the torch oracle's quaternion -> rotation)
    from the documented convention: rotations by theta about each axis turn
    the next axis towards the one after it, and random quaternions give
    scipy's matrix (scipy takes (x, y, z, w))."""
    err = 0.0
    for th in (0.3, 1.1, 2.5, -0.7):
        c, s = math.cos(th / 2), math.sin(th / 2)
        for axis in range(3):
            q = np.zeros(4)
            q[0], q[1 + axis] = c, s
            R = fn(torch.tensor(q)).numpy()
            e_next = np.zeros(3)
            e_next[(axis + 1) % 3] = 1.0
            want = np.zeros(3)
            want[(axis + 1) % 3] = math.cos(th)
            want[(axis + 2) % 3] = math.sin(th)
            err = max(err, np.abs(R @ e_next - want).max())
    q = np.random.default_rng(0).standard_normal((500, 4))
    R = fn(torch.tensor(q)).numpy()
    want = Rotation.from_quat(q[:, [1, 2, 3, 0]]).as_matrix()
    return max(err, np.abs(R - want).max())


def test_quat_to_rotmat_matches_documented_convention():
    assert _quat_rot_error_torch(torch_ref.quat_to_rotmat) < 1e-12


@pytest.mark.parametrize("mutation", ["transposed", "xyzw_order"])
def test_quat_to_rotmat_check_rejects_planted_mistakes(mutation):
    old = "w, x, y, z = torch.unbind(q, dim=-1)"
    new = {"transposed": "w, x, y, z = torch.unbind(q * q.new_tensor([-1.0, 1, 1, 1]), dim=-1)",
           "xyzw_order": "x, y, z, w = torch.unbind(q, dim=-1)"}[mutation]
    fn = _mutated_py(torch_ref, "quat_to_rotmat", old, new)
    assert _quat_rot_error_torch(fn) > 0.1


def _on_axis_conic_error(lib=None, seed=0, n=400):
    """Gaussians of random orientation on the optical axis of an identity
    camera: the 2D covariance is (f/z)^2 times the xy block of
    Sigma = R diag(s^2) R^T (R from scipy) plus eps2d, so the conic is its
    inverse.  Returns the largest error relative to the conic's size."""
    rng = np.random.default_rng(seed)
    f, z, W, H = 300.0, 4.0, 320, 240
    q = rng.standard_normal((n, 4))
    s = np.stack([rng.permutation([0.02, 0.05, 0.1]) for _ in range(n)])
    means = np.tile([0.0, 0.0, z], (n, 1))
    K = np.array([[[f, 0, W / 2], [0, f, H / 2], [0, 0, 1]]])
    with _using_c_oracle(lib):
        out = exact.projection_fwd(means, None, q, s, None, np.eye(4)[None], K, W, H)
    assert out["valid"].all()
    R = Rotation.from_quat(q[:, [1, 2, 3, 0]]).as_matrix()
    Sig = R @ (s[:, :, None] ** 2 * np.swapaxes(R, 1, 2))
    c2 = (f / z) ** 2 * Sig[:, :2, :2] + 0.3 * np.eye(2)
    det = c2[:, 0, 0] * c2[:, 1, 1] - c2[:, 0, 1] ** 2
    want = np.stack([c2[:, 1, 1], -c2[:, 0, 1], c2[:, 0, 0]], -1) / det[:, None]
    got = out["conics"][0].astype(np.float64)
    return (np.abs(got - want).max(-1) / np.abs(want).max(-1)).max()


def test_c_oracle_rotation_matches_documented_convention():
    assert _on_axis_conic_error() < 1e-5


def test_c_oracle_rotation_check_rejects_transposed_rotation(tmp_path):
    # the conjugate quaternion rotates by the transpose
    lib = _mutated_c_oracle(tmp_path, "w = w * inv;", "w = -w * inv;")
    assert _on_axis_conic_error(lib) > 0.05


def test_rotated_anisotropic_gaussian_closed_form():
    """Scales (s1, s2, s3) turned by theta about z, seen on axis: the conic is
    the inverse of (f/z)^2 Rot(theta) diag(s1^2, s2^2) Rot(theta)^T + 0.3 I.
    At 90 degrees the two diagonals swap; at 30 degrees the off-diagonal
    c s (s1^2 - s2^2) (f/z)^2 is positive, so the sense of rotation shows."""
    f, z, W, H = 300.0, 4.0, 320, 240
    s = np.array([[0.1, 0.03, 0.05]])
    K = np.array([[[f, 0, W / 2], [0, f, H / 2], [0, 0, 1]]])
    for deg in (90.0, 30.0):
        th = math.radians(deg)
        q = np.array([[math.cos(th / 2), 0.0, 0.0, math.sin(th / 2)]])
        out = exact.projection_fwd(np.array([[0.0, 0.0, z]]), None, q, s, None,
                                   np.eye(4)[None], K, W, H)
        a, b = (f * s[0, 0] / z) ** 2, (f * s[0, 1] / z) ** 2
        c, sn = math.cos(th), math.sin(th)
        m = np.array([[a * c * c + b * sn * sn, (a - b) * c * sn],
                      [(a - b) * c * sn, a * sn * sn + b * c * c]]) + 0.3 * np.eye(2)
        inv = np.linalg.inv(m)
        np.testing.assert_allclose(out["conics"][0, 0], [inv[0, 0], inv[0, 1], inv[1, 1]],
                                   rtol=1e-5, atol=1e-7)
        if deg == 90.0:
            np.testing.assert_allclose(out["conics"][0, 0, [0, 2]],
                                       [1 / (b + 0.3), 1 / (a + 0.3)], rtol=1e-5)
        else:
            # the conic's b is -cov01/det: negative for a positive cov01
            assert out["conics"][0, 0, 1] < -1e-3


# --------------------------------------------------------------------------
# View matrix (world -> camera)
# --------------------------------------------------------------------------
def _camera_points(R, p, rng, n=50):
    """Points p + a x_c + b y_c + d z_c in front of the camera and their
    camera coordinates (a, b, d)."""
    d = rng.uniform(2.0, 8.0, n)
    a = rng.uniform(-0.4, 0.4, n) * d
    b = rng.uniform(-0.3, 0.3, n) * d
    cam = np.stack([a, b, d], -1)
    return p + cam @ R, cam


def _viewmat_errors(project):
    """Largest |means2d - (c + f (a, b) / d)| in pixels, |depth - d|, and
    conic error of a Gaussian whose axes are the camera's (rotation R^T,
    so its camera-space covariance is diag(s^2)), over several look-at
    cameras.  ``project(means, quats, scales, vm, K, W, H)`` returns
    (means2d [n,2], depths [n], conics [n,3], valid [n])."""
    rng = np.random.default_rng(3)
    f, W, H = 300.0, 320, 240
    K = np.array([[f, 0, W / 2], [0, f, H / 2], [0, 0, 1]])
    e_px = e_d = e_con = 0.0
    s = np.array([0.08, 0.02, 0.05])
    for p in _CAMERA_POSITIONS:
        vm, R = _look_at(p)
        pts, cam = _camera_points(R, np.asarray(p), rng)
        q = np.tile(_wxyz(Rotation.from_matrix(R.T)), (pts.shape[0], 1))
        m2, dep, con, valid = project(pts, q, np.tile(s, (pts.shape[0], 1)), vm, K, W, H)
        if not valid.all():
            # every point lies in front of the camera and inside the image
            return np.inf, np.inf, np.inf
        want = np.stack([W / 2 + f * cam[:, 0] / cam[:, 2],
                         H / 2 + f * cam[:, 1] / cam[:, 2]], -1)
        e_px = max(e_px, np.abs(m2 - want).max())
        e_d = max(e_d, np.abs(dep - cam[:, 2]).max())
        # on the optical axis the conic is diag(1 / ((f s / d)^2 + 0.3))
        on_axis = p + 5.0 * R[2]
        m2a, _, cona, _ = project(on_axis[None], q[:1], s[None], vm, K, W, H)
        wa = np.array([1 / ((f * s[0] / 5) ** 2 + 0.3), 0.0, 1 / ((f * s[1] / 5) ** 2 + 0.3)])
        e_con = max(e_con, np.abs(cona[0] - wa).max() / wa.max())
    return e_px, e_d, e_con


def _project_c(lib=None):
    def project(pts, q, s, vm, K, W, H):
        with _using_c_oracle(lib):
            out = exact.projection_fwd(pts, None, q, s, None, vm[None], K[None], W, H)
        return (out["means2d"][0].astype(np.float64), out["depths"][0].astype(np.float64),
                out["conics"][0].astype(np.float64), out["valid"][0])
    return project


def _project_torch(fn=None):
    fn = fn or torch_ref.projection_ref

    def project(pts, q, s, vm, K, W, H):
        t = lambda a: torch.tensor(np.asarray(a), dtype=torch.float64)
        out = fn(t(pts), None, t(q), t(s), t(vm)[None], t(K)[None], W, H)
        return (out["means2d"][0].numpy(), out["depths"][0].numpy(),
                out["conics"][0].numpy(), out["valid"][0].numpy())
    return project


def test_c_oracle_viewmat_is_world_to_camera():
    e_px, e_d, e_con = _viewmat_errors(_project_c())
    assert e_px < 1e-3 and e_d < 1e-5 and e_con < 1e-4, (e_px, e_d, e_con)


def test_torch_oracle_viewmat_is_world_to_camera():
    e_px, e_d, e_con = _viewmat_errors(_project_torch())
    assert e_px < 1e-9 and e_d < 1e-12 and e_con < 1e-12, (e_px, e_d, e_con)


@pytest.mark.parametrize("mutation", ["transposed_R", "transposed_quat"])
def test_c_oracle_viewmat_check_rejects_planted_mistakes(mutation, tmp_path):
    old, new = {
        "transposed_R": ("R[i * 3 + j] = vm[i * 4 + j];", "R[j * 3 + i] = vm[i * 4 + j];"),
        "transposed_quat": ("w = w * inv;", "w = -w * inv;"),
    }[mutation]
    lib = _mutated_c_oracle(tmp_path, old, new)
    e_px, e_d, e_con = _viewmat_errors(_project_c(lib))
    assert e_px > 1.0 or e_d > 0.1 or e_con > 0.05, (e_px, e_d, e_con)


@pytest.mark.parametrize("mutation", ["transposed_R", "rotated_covariance_once"])
def test_torch_oracle_viewmat_check_rejects_planted_mistakes(mutation):
    old, new = {
        "transposed_R": ("R = viewmats[..., :3, :3]", "R = viewmats[..., :3, :3].mT"),
        "rotated_covariance_once": ('"...cij,...njk,...clk->...cnil", R, Sigma, R',
                                    '"...cij,...njl->...cnil", R, Sigma'),
    }[mutation]
    fn = _mutated_py(torch_ref, "projection_ref", old, new)
    e_px, e_d, e_con = _viewmat_errors(_project_torch(fn))
    assert e_px > 1.0 or e_d > 0.1 or e_con > 0.05, (e_px, e_d, e_con)


# --------------------------------------------------------------------------
# Camera centre and SH view direction
# --------------------------------------------------------------------------
def _centre_error(fn):
    vms = np.stack([_look_at(p)[0] for p in _CAMERA_POSITIONS])
    got = fn(torch.tensor(vms)).numpy()
    return np.abs(got - np.asarray(_CAMERA_POSITIONS)).max()


def test_camera_centre_is_the_camera_position():
    assert _centre_error(torch_ref.camera_centers) < 1e-12
    # the package's own helper for the dense path (rendering.py:216-224)
    from gsplat_amd.rendering import viewmat_to_camera_position
    assert _centre_error(viewmat_to_camera_position) < 1e-12


_CENTRE_MUTATIONS = {
    "minus_R_t": ("-(R.transpose(-1, -2) @ t)", "-(R @ t)"),
    "plus_RT_t": ("-(R.transpose(-1, -2) @ t)", "(R.transpose(-1, -2) @ t)"),
}


@pytest.mark.parametrize("mutation", sorted(_CENTRE_MUTATIONS))
def test_camera_centre_check_rejects_planted_mistakes(mutation):
    fn = _mutated_py(torch_ref, "camera_centers", *_CENTRE_MUTATIONS[mutation])
    assert _centre_error(fn) > 0.1


def _sh_direction_render_error():
    """One Gaussian at the world origin seen by a look-at camera: it lands on
    the centre of pixel (32, 24) (principal point (32.5, 24.5)), so
    alpha = opacity = 0.5 there and the pixel is 0.5 times its colour.  With
    degree-1 SH coefficients that put the three band-1 bases, one per
    channel, the colour is 0.5 + sqrt(3 / 4 pi) (-d_y, d_z, -d_x) for the
    direction d = (origin - camera position) / |.|."""
    p = np.array([3.0, -1.0, 4.0])
    vm, _ = _look_at(p)
    W, H, f = 64, 48, 60.0
    K = torch.tensor([[[f, 0, 32.5], [0, f, 24.5], [0, 0, 1]]])
    coeffs = torch.zeros(1, 4, 3)
    coeffs[0, 1, 0] = coeffs[0, 2, 1] = coeffs[0, 3, 2] = 1.0
    rc, ra, _ = torch_ref.rasterization_ref(
        torch.zeros(1, 3), torch.tensor([[1.0, 0, 0, 0]]), torch.full((1, 3), 0.05),
        torch.tensor([0.5]), coeffs, torch.tensor(vm, dtype=torch.float32)[None], K, W, H,
        sh_degree=1)
    d = -p / np.linalg.norm(p)
    colour = 0.5 + math.sqrt(3 / (4 * math.pi)) * np.array([-d[1], d[2], -d[0]])
    got = rc[0, 24, 32].detach().numpy()
    assert abs(ra[0, 24, 32, 0].item() - 0.5) < 1e-6
    return np.abs(got - 0.5 * colour).max()


def test_sh_view_direction_closed_form():
    assert _sh_direction_render_error() < 1e-6


@pytest.mark.parametrize("mutation", sorted(_CENTRE_MUTATIONS) + ["reversed_direction"])
def test_sh_view_direction_check_rejects_planted_mistakes(mutation, monkeypatch):
    if mutation == "reversed_direction":
        fn = _mutated_py(torch_ref, "rasterization_ref",
                         "dirs = means[g].to(dtype) - campos[c][None, :]",
                         "dirs = campos[c][None, :] - means[g].to(dtype)")
        monkeypatch.setattr(torch_ref, "rasterization_ref", fn)
    else:
        fn = _mutated_py(torch_ref, "camera_centers", *_CENTRE_MUTATIONS[mutation])
        monkeypatch.setattr(torch_ref, "camera_centers", fn)
    assert _sh_direction_render_error() > 1e-2


# --------------------------------------------------------------------------
# Adam moment decay
# --------------------------------------------------------------------------
def _adam_closed_form_error(fn, k=8):
    """k steps of one constant gradient g from moments (m0, v0):
    m_k = b1^k m0 + (1 - b1^k) g, v_k = b2^k v0 + (1 - b2^k) g^2, and the
    parameter moves by -lr m_j / (sqrt(v_j) + eps) at each step j; rows with
    valid = False never change.  Returns the largest relative error."""
    rng = np.random.default_rng(4)
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-15
    g = rng.standard_normal((64, 3)).astype(np.float32)
    m0 = np.where(rng.random((64, 1)) < 0.5, 0.0, rng.standard_normal((64, 3))).astype(np.float32)
    v0 = np.where(rng.random((64, 1)) < 0.5, 0.0, rng.random((64, 3))).astype(np.float32)
    p0 = rng.standard_normal((64, 3)).astype(np.float32)
    valid = rng.random(64) > 0.25
    p, m, v = p0, m0, v0
    for _ in range(k):
        p, m, v = fn(p, g, m, v, valid, lr, b1, b2, eps)
    # the closed form in float64 with the float32 values of the constants
    b1, b2 = float(np.float32(b1)), float(np.float32(b2))
    g64, m64, v64 = g.astype(np.float64), m0.astype(np.float64), v0.astype(np.float64)
    mk = b1 ** k * m64 + (1 - b1 ** k) * g64
    vk = b2 ** k * v64 + (1 - b2 ** k) * g64 ** 2
    dp = np.zeros_like(g64)
    for j in range(1, k + 1):
        mj = b1 ** j * m64 + (1 - b1 ** j) * g64
        vj = b2 ** j * v64 + (1 - b2 ** j) * g64 ** 2
        dp -= lr * mj / (np.sqrt(vj) + eps)
    rel = lambda a, b: (np.abs(a - b) / (np.abs(b) + 1e-30)).max()
    # the parameter to its float32 rounding: relative to the k steps' scale
    err_p = np.abs((p - p0) - dp)[valid].max() / (k * lr)
    err = max(rel(m[valid], mk[valid]), rel(v[valid], vk[valid]), 0.01 * err_p)
    unchanged = (np.array_equal(p[~valid], p0[~valid]) and np.array_equal(m[~valid], m0[~valid])
                 and np.array_equal(v[~valid], v0[~valid]))
    return err if unchanged else np.inf


def test_adam_k_steps_closed_form():
    assert _adam_closed_form_error(exact.adam) < 1e-5


_ADAM_MUTATIONS = {
    "b2_decays_m": ("m_new = b1 * m + (one - b1) * g", "m_new = b2 * m + (one - b1) * g"),
    "b1_decays_v": ("v_new = b2 * v + (one - b2) * g * g", "v_new = b1 * v + (one - b2) * g * g"),
    "betas_swapped": ("m_new = b1 * m + (one - b1) * g", "m_new = b2 * m + (one - b2) * g"),
    "m_weight_b2": ("m_new = b1 * m + (one - b1) * g", "m_new = b1 * m + (one - b2) * g"),
    "v_not_squared": ("(one - b2) * g * g", "(one - b2) * np.abs(g)"),
}


@pytest.mark.parametrize("mutation", sorted(_ADAM_MUTATIONS))
def test_adam_closed_form_rejects_planted_mistakes(mutation):
    fn = _mutated_py(exact, "adam", *_ADAM_MUTATIONS[mutation])
    assert _adam_closed_form_error(fn) > 1e-3
