"""CPU checks of the host side: the C ABI's loadable surface, the ctypes mirror of its structs, argument
validation that returns before any device call, kernel selection, and the plain-PyTorch path of the package
against the oracle. No kernel is launched here."""

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import data
from oracle import reference as ref

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "trnopt_hip.h"


@pytest.fixture(scope="module")
def hk():
    from trnopt import hip_sinkhorn
    hip_sinkhorn.lib()
    return hip_sinkhorn


def test_library_exports_every_declared_symbol(hk):
    declared = set(re.findall(r"\b(sk_[a-z0-9_]+)\s*\(", HEADER.read_text()))
    assert declared, "no declarations found"
    lb = hk.lib()
    missing = sorted(n for n in declared if not hasattr(lb, n))
    assert not missing
    assert declared == set(hk.SYMBOLS)              # the binding covers exactly the header


def test_ctypes_structs_match_the_header(tmp_path):
    """sizeof / offsetof of every ABI struct, from the C compiler, against the ctypes mirror."""
    from trnopt.hip_sinkhorn import SkCloud, SkLoop, SkState
    fields = {"sk_cloud_f32": (SkCloud, [f[0] for f in SkCloud._fields_]),
              "sk_state": (SkState, [f[0] for f in SkState._fields_]),
              "sk_loop_f32": (SkLoop, [f[0] for f in SkLoop._fields_])}
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void) {"]
    for s, (_, names) in fields.items():
        lines.append(f'printf("{s} size %zu\\n", sizeof({s}));')
        for n in names:
            lines.append(f'printf("{s} {n} %zu\\n", offsetof({s}, {n}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out if l}
    for s, (cls, names) in fields.items():
        assert got[(s, "size")] == ctypes.sizeof(cls), s
        for n in names:
            assert got[(s, n)] == getattr(cls, n).offset, (s, n)


def test_constants_match_the_header(hk):
    text = HEADER.read_text()
    const = lambda name: int(re.search(rf"#define {name} (\d+)", text).group(1))   # noqa: E731
    assert hk.TILE == const("SK_TILE") and hk.KP_ALIGN == const("SK_KP_ALIGN") and hk.KP_MAX == const("SK_KP_MAX")
    lb = hk.lib()
    assert lb.sk_version() >= 100
    for n in (1, 31, 32, 33, 10_000, 65_536):
        assert lb.sk_pad_points(n) == hk.pad_points(n)
    for d in (1, 7, 8, 30, 64, 65, 128):
        assert lb.sk_pad_dim(d) == hk.pad_dim(d)
        assert lb.sk_packed_bytes(1000, d) == hk.packed_bytes(1000, d) == 256 + 1024 * hk.pad_dim(d) * 8
    assert lb.sk_packed_bytes(10, 129) == 0 and lb.sk_packed_bytes(0, 8) == 0


def test_rejected_arguments_return_codes_not_aborts(hk):
    """Validation that happens before any device call: null pointers, shapes, the dimension limit."""
    lb = hk.lib()
    assert lb.sk_half_step_f32(None, None, None, 32, None, None, None, 32, 4, 0, None, None, None, None, None, 1,
                               None, 0, None) == -1
    assert b"null pointer" in lb.sk_last_error()
    fake = 4096   # a non-null address that is never dereferenced: validation fails first
    assert lb.sk_row_lse_f32(fake, fake, fake, 10, 10, 200, fake, 1 << 20, None) == -2
    assert b"SK_KP_MAX" in lb.sk_last_error()
    assert lb.sk_row_lse_f32(fake, fake, fake, 0, 10, 8, fake, 1 << 20, None) == -2
    assert lb.sk_pack_cloud_f32(None, 10, 4, 4, None, None) == -1
    assert lb.sk_pack_cloud_f32(fake, 10, 8, 4, fake, None) == -2          # ld < d
    assert lb.sk_pack_cloud_f32(fake, 10, 4, 4, fake + 8, None) == -1      # out not 16-byte aligned
    assert lb.sk_loop_init_f32(None, None) == -1
    assert lb.sk_loop_run_f32(None, 1, None) == -1


def test_half_step_shape_rules(hk):
    lb = hk.lib()
    fake = 4096
    # rows_pad not a multiple of 32
    assert lb.sk_half_step_f32(fake, fake, None, 33, fake, fake + 256, fake, 32, 4, 0, fake, None, fake + 512, None,
                               None, 1, fake, 1 << 20, None) == -2
    # fh aliasing gh
    assert lb.sk_half_step_f32(fake, fake, None, 32, fake, fake, fake, 32, 4, 0, fake, None, fake, None, None, 1,
                               fake, 1 << 20, None) == -1
    # meas without w
    assert lb.sk_half_step_f32(fake, fake, None, 32, fake, fake + 256, fake, 32, 4, 0, fake, None, fake + 512, fake,
                               None, 1, fake, 1 << 20, None) == -1
    # rows_role other than 0 / 1
    assert lb.sk_half_step_f32(fake, fake, None, 32, fake, fake + 256, fake, 32, 4, 2, fake, None, fake + 512, None,
                               None, 1, fake, 1 << 20, None) == -1
    assert b"rows_role" in lb.sk_last_error()


def test_noalloc_half_step_validates_like_the_workspace_entry_point(hk):
    """sk_half_step_noalloc_f32 applies sk_half_step_f32's checks and refuses shapes whose partial slots would
    not fit its static scratch (SK_NOALLOC_SCRATCH_BYTES), all before any device call."""
    lb = hk.lib()
    fake = 4096
    limit = int(re.search(r"#define SK_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", HEADER.read_text())
                .group(1)) << 20
    assert limit == 16 << 20
    assert lb.sk_half_step_noalloc_f32(None, None, None, 32, None, None, None, 32, 4, 0, None, None, None, None, None,
                                       1, None) == -1
    assert lb.sk_half_step_noalloc_f32(fake, fake, None, 33, fake, fake + 256, fake, 32, 4, 0, fake, None, fake + 512,
                                       None, None, 1, None) == -2
    assert lb.sk_half_step_noalloc_f32(fake, fake, None, 32, fake, fake, fake, 32, 4, 0, fake, None, fake, None, None,
                                       1, None) == -1
    rows_pad = (1 << 21) + 32                      # one slot per row: 8 bytes x rows_pad > 16 MiB
    assert lb.sk_half_step_workspace_bytes(rows_pad, 32, 4) > limit
    assert lb.sk_half_step_noalloc_f32(fake, fake, None, rows_pad, fake, fake + 256, fake, 32, 4, 0, fake, None,
                                       fake + 512, None, None, 1, None) == -3
    assert b"static scratch" in lb.sk_last_error()


def _pass_cost(rows_pad, m_pad, kp):
    """A pass's length on its split's cost line: row groups (256 rows) x column tiles (32), plus the cost of each
    row-group boundary (6 tiles up to kp 64, 4 above: make_plan)."""
    ngroups, nt = -(-rows_pad // 256), m_pad // 32
    return ngroups * nt + (6 if kp <= 64 else 4) * (ngroups - 1)


def _smallest_even_share(costs, total):
    """The smallest per-workgroup cost T at which one workgroup per ceil(cost / T) tiles (one at least) fits
    `total` workgroups, by bisection over T."""
    need = lambda T: sum(max(1, -(-c // T)) for c in costs)       # noqa: E731
    lo, hi = 1, max(costs)
    while lo < hi:
        mid = (lo + hi) // 2
        lo, hi = (lo, mid) if need(mid) <= total else (mid + 1, hi)
    return lo


@pytest.mark.parametrize("count,d", [(1, 64), (1, 30), (2, 30), (5, 128), (38, 30), (300, 16)])
def test_batch_plan_shares_the_workgroups_by_work(hk, count, d):
    """sk_loop_batch_plan (host arithmetic, no device call): each loop's f and g pass get workgroups so that no
    workgroup carries more tiles than the smallest even share T of the 256 CUs, at least one each, every CU used
    while a pass has more tiles than workgroups; one loop gets the split of its own launches, min(256, tiles)."""
    lb = hk.lib()
    rng = np.random.default_rng(count + d)
    sizes = np.exp(rng.uniform(np.log(2), np.log(9000), size=(count, 2))).astype(int)
    nx = [hk.pad_points(int(a)) for a, _ in sizes]
    ny = [hk.pad_points(int(b)) for _, b in sizes]
    kp = hk.pad_dim(d)
    wg = (ctypes.c_int * (2 * count))()
    assert lb.sk_loop_batch_plan((ctypes.c_int * count)(*nx), (ctypes.c_int * count)(*ny), count, d, wg) == 0
    for side, costs in ((0, [_pass_cost(nx[k], ny[k], kp) for k in range(count)]),
                        (1, [_pass_cost(ny[k], nx[k], kp) for k in range(count)])):
        P = [wg[2 * k + side] for k in range(count)]
        assert min(P) >= 1 and all(P[k] <= max(1, costs[k]) for k in range(count))
        if count <= 256:
            assert sum(P) == min(256, sum(costs))
        else:
            assert P == [1] * count
        T = _smallest_even_share(costs, 256)
        assert max(-(-c // p) for c, p in zip(costs, P)) <= T
        if count == 1:
            assert P == [min(256, costs[0])]


def test_batch_entry_points_validate_before_any_device_call(hk):
    lb = hk.lib()
    assert lb.sk_loop_batch_workspace_bytes(0) == 0 and lb.sk_loop_batch_workspace_bytes(1025) == 0
    one = lb.sk_loop_batch_workspace_bytes(1)
    assert 0 < one < lb.sk_loop_batch_workspace_bytes(38)
    ints = (ctypes.c_int * 2)(64, 64)
    out = (ctypes.c_int * 4)()
    assert lb.sk_loop_batch_plan(None, ints, 1, 30, out) == -1
    assert lb.sk_loop_batch_plan(ints, ints, 0, 30, out) == -2
    assert lb.sk_loop_batch_plan(ints, ints, 1, 200, out) == -2                 # d beyond SK_KP_MAX
    assert lb.sk_loop_batch_plan((ctypes.c_int * 1)(40), ints, 1, 30, out) == -2   # not a multiple of 32
    loops = (ctypes.POINTER(hk.SkLoop) * 1)(ctypes.pointer(hk.SkLoop()))
    launch = (ctypes.c_int * 3)()
    assert lb.sk_loop_batch_init_f32(None, 1, 4096, one, launch, None) == -1
    assert lb.sk_loop_batch_init_f32(loops, 0, 4096, one, launch, None) == -2
    assert lb.sk_loop_batch_init_f32(loops, 1, 4096, one - 1, launch, None) == -3
    assert lb.sk_loop_batch_init_f32(loops, 1, 4096 + 16, one, launch, None) == -1   # misaligned
    assert lb.sk_loop_batch_init_f32(loops, 1, 4096, one, launch, None) == -1        # the loop's null pointers
    assert lb.sk_loop_run_batch_f32(4096, one, 1, (ctypes.c_int * 3)(2, 0, 5), 1, None) == -1
    assert lb.sk_loop_run_batch_f32(4096, one, 1, (ctypes.c_int * 3)(9, 5, 5), 1, None) == -1   # kp 144
    assert lb.sk_loop_run_batch_f32(4096, one, 1, (ctypes.c_int * 3)(2, 5, 2000), 1, None) == -1
    assert lb.sk_loop_run_batch_f32(4096, one - 1, 1, (ctypes.c_int * 3)(2, 5, 5), 1, None) == -3
    assert lb.sk_loop_run_batch_f32(4096, one, 1, (ctypes.c_int * 3)(2, 5, 5), -1, None) == -1
    assert b"iters" in lb.sk_last_error()


# ---------------------------------------------------------------------------------------------------------
# Selection and validation of the Python API (src/trnopt/sinkhorn.py:196-208, 254-276; backend.py:30-48)

def test_selection_errors():
    from trnopt import Backend, SinkhornOptions, sinkhorn
    x, y = data.clouds(n=20, m=15, d=3)
    with pytest.raises(ValueError, match="kernel='hip'"):
        sinkhorn(x, y, opts=SinkhornOptions(kernel="hip"))                   # CPU backend
    if not torch.cuda.is_available():
        with pytest.raises(ValueError, match="kernel='hip'"):
            sinkhorn(x, y, opts=SinkhornOptions(kernel="hip", backend=Backend.preset("rocm")))
    with pytest.raises(ValueError, match="nki"):
        sinkhorn(x, y, opts=SinkhornOptions(kernel="nki"))
    with pytest.raises(ValueError, match="unknown kernel"):
        sinkhorn(x, y, opts=SinkhornOptions(kernel="cuda"))
    with pytest.raises(ValueError, match="cores"):
        sinkhorn(x, y, opts=SinkhornOptions(cores=2))
    with pytest.raises(ValueError, match="unknown backend preset"):
        Backend.preset("tpu")


def test_input_validation():
    from trnopt import SinkhornOptions, sinkhorn
    x, y = data.clouds(n=20, m=15, d=3)
    with pytest.raises(ValueError, match="sum"):
        sinkhorn(x, y, a=np.full(20, 0.1))
    with pytest.raises(ValueError, match="pass rho"):
        sinkhorn(x, y, a_target=np.full(20, 0.05))
    with pytest.raises(ValueError, match="positive"):
        sinkhorn(x, y, a=-np.full(20, 0.05), opts=SinkhornOptions(rho=1.0))
    with pytest.raises(ValueError, match="positive"):
        sinkhorn(x, y, b=np.full(14, 1 / 14), opts=SinkhornOptions(rho=1.0))
    with pytest.raises(ValueError, match="same d"):
        sinkhorn(x, y[:, :2])
    with pytest.raises(ValueError, match="2-D"):
        sinkhorn(x[:, 0], y)
    with pytest.raises(ValueError, match="at least one point"):
        sinkhorn(x[:0], y, opts=SinkhornOptions(rho=1.0, normalize=False))
    with pytest.raises(ValueError, match="at least one point"):
        sinkhorn(x, y[:0], opts=SinkhornOptions(rho=1.0, normalize=False))


def test_presets():
    from trnopt import Backend
    r = Backend.preset("rocm")
    assert r.device == "cuda" and r.dtype == torch.float32 and not r.compile
    assert Backend.preset("cpu").dtype == torch.float64
    assert Backend.preset("rocm", compile=True).compile


def test_auto_kernel_is_torch_off_gpu():
    from trnopt import Backend, SinkhornOptions
    from trnopt.sinkhorn import _use_hip
    assert not _use_hip(SinkhornOptions(), 8)
    assert not _use_hip(SinkhornOptions(backend=Backend.preset("cpu-float32")), 8)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("kw", [dict(eps=0.1, tol=1e-6), dict(eps=0.1, rho=(1.0, 5.0), block=40),
                                dict(eps=0.05, eps_start=1.0, tol=1e-5, block=32, block_y=50),
                                dict(eps=0.1, rho=2.0, eps_stages=(1.0, 0.5), check_every=5, normalize="median")])
def test_torch_path_equals_oracle(dtype, kw):
    """kernel="torch" of the package runs the reference's op sequence: identical to the oracle, bit for bit."""
    from trnopt import Backend, SinkhornOptions, sinkhorn
    x, y = data.clouds(n=137, m=91, d=5)
    be = Backend.preset("cpu", dtype=dtype)
    r = sinkhorn(x, y, opts=SinkhornOptions(kernel="torch", backend=be, max_iters=3000, **kw))
    o = ref.sinkhorn_ref(x, y, max_iters=3000, dtype=dtype, **kw)
    assert r.iterations == o.iterations and r.converged == o.converged
    np.testing.assert_array_equal(r.f, o.f)
    np.testing.assert_array_equal(r.g, o.g)
    if r.row_mass is not None:
        np.testing.assert_array_equal(r.row_mass, o.row_mass)
        np.testing.assert_array_equal(r.col_mass, o.col_mass)
