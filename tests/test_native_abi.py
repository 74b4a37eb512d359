"""The C ABI library (include/morphocore_amd.h): it loads, exports every declared symbol, and its
argument validation answers with the reference's messages — all without a GPU (validation returns
before any HIP call)."""
import ctypes
import os
import re

import pytest

from morphocore_amd import _native

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "morphocore_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(mca_\w+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _native.lib()
    symbols = declared_symbols()
    assert len(symbols) == 59
    for name in symbols:
        assert hasattr(lib, name), name
    assert sorted(_native.EXPORTS) == symbols


def test_version():
    assert _native.version().startswith("0.13.1")


GEOM = (2, 3, 4, 3, 16, 16, 3, 3)  # B, Cin, Cout, Cw, H, W, KH, KW


def _forward(merge=2, geom=GEOM, op=0, indices=None):
    lib = _native.lib()
    return lib.mca_morpho_forward_f32(op, merge, 0, 0.0, None, None, 0, None, indices, *geom, None)


@pytest.mark.parametrize("merge,message", [(9, "Unknown merge mode 9"), (-1, "Unknown merge mode -1"), (4, "Unsupported merge operation")])
def test_rejects_merge(merge, message):
    assert _forward(merge) == 1
    assert _native.lib().mca_last_error().decode() == message


def test_rejects_identity_shapes():
    assert _forward(5, (2, 3, 4, 1, 8, 8, 3, 3)) == 1
    assert "Identity mode requires weight.shape[0] == input.shape[1]" in _native.lib().mca_last_error().decode()
    assert _forward(5, (2, 3, 3, 3, 8, 8, 3, 3)) == 1
    assert "Identity mode requires weight.shape[1] == 1" in _native.lib().mca_last_error().decode()


def test_rejects_channel_mismatch_and_operation():
    assert _forward(2, (2, 3, 4, 2, 8, 8, 3, 3)) == 1
    assert "Input channels must match weight input channels" in _native.lib().mca_last_error().decode()
    assert _forward(2, op=7) == 1
    assert "Unknown morphological operation" in _native.lib().mca_last_error().decode()


def test_rejects_index_capacity():
    # A non-null indices pointer for a 257 x 257 structuring element (taps >= 65536).
    dummy = ctypes.c_void_p(16)
    assert _forward(0, (1, 1, 1, 1, 8, 8, 257, 257), indices=dummy) == 1
    assert "too large to save indices" in _native.lib().mca_last_error().decode()


def test_indices_bytes():
    lib = _native.lib()
    B, Cin, Cout, Cw, H, W, KH, KW = GEOM
    assert lib.mca_morpho_indices_bytes(0, *GEOM) == B * Cout * H * W * 4  # packed int32 winners
    assert lib.mca_morpho_indices_bytes(2, *GEOM) == B * Cout * Cin * H * W  # one tap byte per pair
    assert lib.mca_morpho_indices_bytes(5, 2, 3, 3, 1, 16, 16, 3, 3) == 2 * 3 * 16 * 16
    assert lib.mca_morpho_indices_bytes(3, 1, 2, 2, 2, 4, 4, 17, 17) == 1 * 2 * 2 * 4 * 4 * 2  # 289 taps: uint16


def test_rejects_too_large_structuring_element_for_lds():
    assert _forward(2, (1, 1, 1, 1, 8, 8, 200, 200)) == 1
    assert "too large" in _native.lib().mca_last_error().decode()


def test_workspace_sizes_and_rejection():
    lib = _native.lib()
    for merge in (0, 1, 2, 3):
        assert lib.mca_morpho_backward_workspace_size_f32(merge, 0, *GEOM) > 0
    assert lib.mca_morpho_backward_workspace_size_f32(0, 1, *GEOM) < lib.mca_morpho_backward_workspace_size_f32(0, 0, *GEOM)
    assert lib.mca_morpho_backward_workspace_size_f64(2, 0, *GEOM) > lib.mca_morpho_backward_workspace_size_f32(2, 0, *GEOM)
    assert lib.mca_morpho_backward_workspace_size_f32(9, 0, *GEOM) == 0
    for merge in (0, 2, 3, 1):
        assert lib.mca_smorph_backward_workspace_size_f32(merge, *GEOM) > 0
    # A workspace that is too small is an argument error, before any device work.
    rc = lib.mca_morpho_backward_f32(0, 2, 0, 0.0, None, None, 0, None, None, None, None, *GEOM, None, 16, None)
    assert rc == 1 and "Workspace too small" in lib.mca_last_error().decode()
    rc = lib.mca_smorph_backward_f32(2, None, None, None, None, None, None, None, None, *GEOM, None, 16, None)
    assert rc == 1 and "Workspace too small" in lib.mca_last_error().decode()


def test_smorph_stats_bytes_and_rejection():
    """The saved-statistics entry points: three float32 values per channel pair and output pixel for
    the static sizes, none otherwise; a configuration without them, or a null buffer, is an argument
    error before any device work."""
    lib = _native.lib()
    B, Cin, Cout, Cw, H, W = 2, 3, 4, 3, 16, 16
    for k in (3, 5, 7, 11):
        assert lib.mca_smorph_stats_bytes_f32(2, B, Cin, Cout, Cw, H, W, k, k) == 12 * B * Cout * Cin * H * W
    assert lib.mca_smorph_stats_bytes_f32(5, 2, 3, 3, 1, H, W, 7, 7) == 12 * 2 * 3 * H * W  # IDENTITY: one pair per output
    assert lib.mca_smorph_stats_bytes_f32(2, B, Cin, Cout, Cw, H, W, 4, 4) == 0
    assert lib.mca_smorph_stats_bytes_f32(2, B, Cin, Cout, Cw, H, W, 3, 5) == 0
    assert lib.mca_smorph_stats_bytes_f32(9, B, Cin, Cout, Cw, H, W, 3, 3) == 0
    rc = lib.mca_smorph_forward_stats_f32(2, None, None, None, None, None, B, Cin, Cout, Cw, H, W, 4, 4, None)
    assert rc == 1 and "No saved smorph statistics" in lib.mca_last_error().decode()
    rc = lib.mca_smorph_forward_stats_f32(2, None, None, None, None, None, B, Cin, Cout, Cw, H, W, 3, 3, None)
    assert rc == 1 and "stats must not be null" in lib.mca_last_error().decode()
    rc = lib.mca_smorph_backward_stats_f32(2, None, None, None, None, None, None, None, None, None, B, Cin, Cout, Cw, H, W, 3, 3,
                                           None, 0, None)
    assert rc == 1 and "stats must not be null" in lib.mca_last_error().decode()
    assert _native.smorph_stats_bytes(2, __import__("torch").float64, (B, Cin, Cout, Cw, H, W, 3, 3)) == 0
    # An empty batch has no statistics to save: accepted without a buffer, and nothing is launched.
    assert lib.mca_smorph_stats_bytes_f32(2, 0, Cin, Cout, Cw, H, W, 3, 3) == 0
    rc = lib.mca_smorph_forward_stats_f32(2, None, None, None, None, None, 0, Cin, Cout, Cw, H, W, 3, 3, None)
    assert rc == 0, lib.mca_last_error().decode()


def test_smorph_scm_stats_bytes_and_rejection():
    """The SMOOTH merge's saved-statistics entry points: as many values as the SUM merge's (three per
    channel pair and output pixel) for the static sizes, none otherwise; a configuration without
    them, or a null buffer, is an argument error before any device work; an empty batch needs none."""
    lib = _native.lib()
    B, Cin, Cout, H, W = 2, 3, 4, 16, 16
    for k in (3, 5, 7, 11):
        assert lib.mca_smorph_scm_stats_bytes_f32(B, Cin, Cout, Cin, H, W, k, k) == 12 * B * Cout * Cin * H * W
    assert lib.mca_smorph_scm_stats_bytes_f32(B, Cin, Cout, Cin, H, W, 4, 4) == 0
    assert lib.mca_smorph_scm_stats_bytes_f32(B, Cin, Cout, Cin, H, W, 3, 5) == 0
    assert lib.mca_smorph_scm_stats_bytes_f32(B, Cin, Cout, 1, H, W, 3, 3) == 0  # Cw != Cin
    nulls = (None,) * 7
    rc = lib.mca_smorph_scm_forward_stats_f32(*nulls, B, Cin, Cout, Cin, H, W, 4, 4, None)
    assert rc == 1 and "No saved smorph statistics" in lib.mca_last_error().decode()
    rc = lib.mca_smorph_scm_forward_stats_f32(*nulls, B, Cin, Cout, Cin, H, W, 3, 3, None)
    assert rc == 1 and "stats must not be null" in lib.mca_last_error().decode()
    rc = lib.mca_smorph_scm_backward_stats_f32(*(None,) * 12, B, Cin, Cout, Cin, H, W, 3, 3, None, 0, None)
    assert rc == 1 and "stats must not be null" in lib.mca_last_error().decode()
    assert _native.smorph_scm_stats_bytes(__import__("torch").float64, (B, Cin, Cout, Cin, H, W, 3, 3)) == 0
    assert lib.mca_smorph_scm_stats_bytes_f32(0, Cin, Cout, Cin, H, W, 3, 3) == 0
    rc = lib.mca_smorph_scm_forward_stats_f32(*nulls, 0, Cin, Cout, Cin, H, W, 3, 3, None)
    assert rc == 0, lib.mca_last_error().decode()


def _smorph_saved_plan_bytes(merge, B, Cin, Cout, H, W, K):
    """Workspace bytes of the float32 smorph backward from saved statistics (two output rows per
    wave: 64 x 8 tiles), for a square static element: slot partials of grad_weight and grad_alpha
    (and for SMOOTH, merge 4, of grad_beta: Cin rows of Cout values per slot), MAX / MIN counts and
    merge target, and the two-stage slot reduction's scratch."""
    align = lambda v: (v + 255) // 256 * 256  # noqa: E731
    ntiles = -(-W // 64) * -(-H // 8)
    nstrips = min(max(-(-8192 // (B * Cin)), 1), ntiles)
    wnumel, npairs = Cout * Cin * K * K, Cout * Cin
    while nstrips > 1 and B * nstrips * (wnumel + npairs) * 4 > (256 << 20):
        nstrips = (nstrips + 1) // 2
    tps = -(-ntiles // nstrips)
    nslots = B * -(-ntiles // tps)
    counts = 2 * B * Cout * H * W * 4 if merge in (0, 1) else 0
    scratch = -(-nslots // 32) * max(wnumel, npairs) * 4 if nslots > 32 else 0
    part_b = nslots * npairs * 4 if merge == 4 else 0
    if merge == 4 and nslots * Cin > 32:
        scratch = max(scratch, -(-(nslots * Cin) // 32) * Cout * 4)
    return align(nslots * wnumel * 4) + align(nslots * npairs * 4) + align(part_b) + align(counts) + align(scratch)


@pytest.mark.parametrize("merge", [0, 2, 3, 4])
@pytest.mark.parametrize("geom", [(4, 64, 100, 100, 3), (4, 64, 100, 100, 7), (2, 16, 300, 300, 5), (1, 8, 160, 200, 11)])
def test_smorph_workspace_covers_the_saved_statistics_plan(merge, geom):
    """The workspace size the caller allocates must also hold the layout of the backward from saved
    statistics, whose rounding of tiles per strip can give more slots than the recomputing plan
    (4 x 64 x 100 x 100: 26 strips against 25). Regression test of an out-of-bounds layout; merge 4
    is the SMOOTH merge's (smorph_scm) backward."""
    B, C, H, W, K = geom
    lib = _native.lib()
    if merge == 4:
        have = lib.mca_smorph_scm_backward_workspace_size_f32(B, C, C, C, H, W, K, K)
    else:
        have = lib.mca_smorph_backward_workspace_size_f32(merge, B, C, C, C, H, W, K, K)
    assert have >= _smorph_saved_plan_bytes(merge, B, C, C, H, W, K)


def test_noalloc_backward_rejects_problems_beyond_its_scratch():
    """The no-allocation backward refuses, before any device work, a problem whose workspace exceeds
    the library's per-GPU scratch (here: configs[4]'s first layer without saved winners)."""
    lib = _native.lib()
    geom = (8, 64, 64, 64, 512, 512, 11, 11)
    assert lib.mca_morpho_backward_workspace_size_f32(0, 0, *geom) > _native.NOALLOC_SCRATCH_BYTES
    rc = lib.mca_morpho_backward_noalloc_f32(0, 0, 1, 0.0, None, None, 0, None, None, None, None, *geom, None)
    assert rc == 1
    assert "Problem too large for the no-allocation backward" in lib.mca_last_error().decode()
    rc = lib.mca_morpho_backward_noalloc_f32(0, 9, 1, 0.0, None, None, 0, None, None, None, None, *GEOM, None)
    assert rc == 1 and lib.mca_last_error().decode() == "Unknown merge mode 9"


def test_pair_supported_sizes():
    lib = _native.lib()
    assert [k for k in range(1, 13) if lib.mca_morpho_pair_supported(k, k)] == [3, 5, 7]
    assert not lib.mca_morpho_pair_supported(3, 5)
    assert not lib.mca_morpho_pair_supported(-3, -3)


def test_pair_rejects_bad_arguments():
    lib = _native.lib()
    pg = (2, 3, 16, 16, 3, 3)
    assert lib.mca_morpho_pair_forward_f32(4, 0, 0.0, 0.0, None, None, None, 0, None, None, None, *pg, None) == 1
    assert "Unknown morphological operation 4" in lib.mca_last_error().decode()
    assert lib.mca_morpho_pair_forward_f32(1, 0, 0.0, 0.0, None, None, None, 0, None, None, None, 2, 3, 16, 16, 9, 9, None) == 1
    assert "3x3, 5x5 or 7x7" in lib.mca_last_error().decode()
    assert lib.mca_morpho_pair_forward_f32(1, 0, 0.0, 0.0, None, None, None, 0, None, ctypes.c_void_p(16), None, *pg, None) == 1
    assert "both be given or both be NULL" in lib.mca_last_error().decode()
    assert lib.mca_morpho_pair_backward_f32(1, None, None, None, None, None, None, *pg, None, 0, None) == 1
    assert "saved taps" in lib.mca_last_error().decode()
    need = lib.mca_morpho_pair_backward_workspace_size_f32(*pg)
    assert need > 0 and lib.mca_morpho_pair_backward_workspace_size_f64(*pg) > need
    assert lib.mca_morpho_pair_backward_workspace_size_f32(2, 3, 16, 16, 4, 4) == 0
    t = ctypes.c_void_p(16)
    assert lib.mca_morpho_pair_backward_f32(1, t, t, None, None, None, None, *pg, None, need - 1, None) == 1
    assert "Workspace too small" in lib.mca_last_error().decode()


def test_sigma_rejects_bad_arguments():
    lib = _native.lib()
    pg = (2, 3, 16, 16, 3, 3)
    inf = float("inf")
    args = lambda fe, fd: (0, fe, fd, None, None, None, 0, None, None, None, None, *pg, None)  # noqa: E731
    assert lib.mca_morpho_sigma_forward_f32(*args(1.0, 2.0)) == 1
    assert "one border value for both operations" in lib.mca_last_error().decode()
    assert lib.mca_morpho_sigma_forward_f32(*args(-inf, inf)) == 1
    assert lib.mca_morpho_sigma_forward_f32(0, 0.0, 0.0, None, None, None, 0, None, None, ctypes.c_void_p(16), None, *pg, None) == 1
    assert "both be given or both be NULL" in lib.mca_last_error().decode()
    assert lib.mca_morpho_sigma_forward_f64(0, 0.0, 0.0, None, None, None, 0, None, None, None, None, 2, 3, 16, 16, 9, 9, None) == 1
    assert "3x3, 5x5 or 7x7" in lib.mca_last_error().decode()
    need = lib.mca_morpho_sigma_backward_workspace_size_f32(*pg)
    assert need > 0 and lib.mca_morpho_sigma_backward_workspace_size_f32(2, 3, 16, 16, 3, 5) == 0
    t = ctypes.c_void_p(16)
    common = (None, None, None, 0, None)
    assert lib.mca_morpho_sigma_backward_f32(0, inf, -inf, *common, None, None, None, None, None, None, None, *pg, None, need, None) == 1
    assert "saved taps" in lib.mca_last_error().decode()
    assert lib.mca_morpho_sigma_backward_f32(0, inf, -inf, *common, t, t, None, None, None, None, None, *pg, None, need - 1, None) == 1
    assert "Workspace too small" in lib.mca_last_error().decode()


def test_rejects_planes_beyond_32_bit_offsets():
    assert _forward(2, (1, 1, 1, 1, 65536, 32768, 3, 3)) == 1
    assert "2^31 - 1 pixels" in _native.lib().mca_last_error().decode()


@pytest.mark.parametrize("merge", [0, 2, 3, 5])
def test_smorph_backward_takes_large_elements(merge):
    """A 31x31 smorph element has a backward (a non-zero workspace) in float32 and float64, also for the
    SMOOTH merge, even within the smallest per-workgroup LDS a device may report (64 KiB: the value
    assumed without a device): the generic kernel takes one output row per wave there. The reference's
    CPU path takes any size (smorph_cpu_kernels.hxx:30-147)."""
    lib = _native.lib()
    B, C, H, W, K = 2, 3, 40, 70, 31
    cw = 1 if merge == 5 else C
    assert lib.mca_smorph_backward_workspace_size_f32(merge, B, C, C, cw, H, W, K, K) > 0
    assert lib.mca_smorph_backward_workspace_size_f64(merge, B, C, C, cw, H, W, K, K) > 0
    assert lib.mca_smorph_scm_backward_workspace_size_f32(B, C, C, C, H, W, K, K) > 0
    assert lib.mca_smorph_scm_backward_workspace_size_f64(B, C, C, C, H, W, K, K) > 0


def test_size_queries_with_empty_dimensions():
    """Every workspace and buffer size query answers for an empty batch, image height or width and for
    no input or output channel (none divides by an empty dimension: an empty smorph batch once stopped
    the process with a division by zero), and the byte counts of empty results are 0."""
    lib = _native.lib()
    base = dict(B=2, Cin=3, Cout=4, H=16, W=16)
    cases = [(), ("B",), ("Cin",), ("Cout",), ("H",), ("W",), ("B", "Cin"), ("H", "W"), ("Cin", "Cout")]
    for zero in cases:
        d = dict(base, **{z: 0 for z in zero})
        for K in (3, 7, 11, 31):
            for merge in (0, 1, 2, 3, 5):
                cin = d["Cin"]
                cout = cin if merge == 5 else d["Cout"]
                cw = 1 if merge == 5 else cin
                g = (d["B"], cin, cout, cw, d["H"], d["W"], K, K)
                lib.mca_morpho_indices_bytes(merge, *g)
                for sfx in ("f32", "f64", "f16", "bf16"):
                    for has_idx in (0, 1):
                        getattr(lib, f"mca_morpho_backward_workspace_size_{sfx}")(merge, has_idx, *g)
                for sfx in ("f32", "f64"):
                    getattr(lib, f"mca_smorph_backward_workspace_size_{sfx}")(merge, *g)
                stats = lib.mca_smorph_stats_bytes_f32(merge, *g)
                if d["B"] * cout * cin * d["H"] * d["W"] == 0:
                    assert stats == 0
            g = (d["B"], d["Cin"], d["Cout"], d["Cin"], d["H"], d["W"], K, K)
            for sfx in ("f32", "f64"):
                getattr(lib, f"mca_smorph_scm_forward_workspace_size_{sfx}")(*g)
                getattr(lib, f"mca_smorph_scm_backward_workspace_size_{sfx}")(*g)
                getattr(lib, f"mca_morpho_pair_backward_workspace_size_{sfx}")(d["B"], d["Cin"], d["H"], d["W"], K, K)
                getattr(lib, f"mca_morpho_sigma_backward_workspace_size_{sfx}")(d["B"], d["Cin"], d["H"], d["W"], K, K)
            lib.mca_smorph_scm_stats_bytes_f32(*g)
