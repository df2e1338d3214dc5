"""The C ABI libraries load without a GPU, export every entry point that
include/*.h declares, and its struct layouts match the reference contracts
(HybridInputRec 128 B, HybridS2S3Config 4616 B with preds at 3968,
HybridS2S3OutputSlot 392 B, GpuTimingSlot 40 B).  No compute call here."""
import ctypes
import re
from pathlib import Path

from ssla_hip import abi, lib

ROOT = Path(__file__).resolve().parent.parent


def declared(header: str, prefix: str = "ssla_hip_"):
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"\w+)\s*\(", text)))


def test_producer_libraries_export_every_declared_symbol():
    from ssla_hip import producer
    g = producer.load_to_gpu()
    names = declared("stage01_to_gpu.h", "s01g_")
    assert len(names) == 18 and sorted(producer.EXPORTED_TO_GPU) == names
    for n in names:
        assert hasattr(g, n), n
    c = producer.load_capi()
    names = declared("stage01_capi.h", "s0_")
    assert len(names) == 5 and sorted(producer.EXPORTED_CAPI) == names
    for n in names:
        assert hasattr(c, n), n


def test_library_exports_every_declared_symbol():
    L = lib.load()
    names = declared("ssla_hip.h")
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), n
    assert sorted(lib.EXPORTED) == names


def test_layout_matches_mirror():
    lib.check_layout()
    lay = lib.layout()
    assert lay["HybridInputRec"] == 128
    assert lay["HybridS2S3Config"] == 4616 and lay["preds_offset"] == 3968
    assert lay["HybridS2S3OutputSlot"] == 392 and lay["GpuTimingSlot"] == 40
    assert abi.HybridS2S3Config.hidden.offset == 8 * 4 + 16 * 32 + 16 * 4 * 40


def test_errors_do_not_cross_the_boundary():
    L = lib.load()
    assert L.ssla_hip_drain_n(None, None, None, None, None) < 0
    assert b"null" in L.ssla_hip_last_error()
    m = ctypes.c_void_p()
    assert L.ssla_hip_model_load(b"/nonexistent/dir", ctypes.byref(m)) < 0
    assert not m.value


def test_two_ring_drain_and_reserve_reject_bad_arguments():
    """ssla_hip_drain_n2 is the two-ring form: any other block count is an
    argument error, reported before any device work (no GPU needed)."""
    L = lib.load()
    cfg = abi.HybridS2S3Config()
    cfg.H2, cfg.W2, cfg.H3, cfg.W3 = 16, 20, 8, 10
    for nb in (0, 1, 3, 16):
        cfg.n_blocks = nb
        rc = L.ssla_hip_drain_n2(ctypes.byref(cfg), None, None, 0, 0, None, None)
        assert rc == abi.SSLA_ERR_ARG, nb
        assert b"n_blocks == 2" in L.ssla_hip_last_error()
    assert L.ssla_hip_drain_n2(None, None, None, 0, 0, None, None) == abi.SSLA_ERR_ARG
    cfg.n_blocks = 1
    assert L.ssla_hip_drain_reserve(ctypes.byref(cfg), -1) == abi.SSLA_ERR_ARG
    cfg.n_blocks = 17
    assert L.ssla_hip_drain_reserve(ctypes.byref(cfg), 10) == abi.SSLA_ERR_ARG
    assert L.ssla_hip_drain_reserve(None, 10) == abi.SSLA_ERR_ARG


def test_constants_match_the_header():
    """Return codes, phase counts and prediction constants of ssla_hip.h
    against the Python mirror."""
    import re
    text = (ROOT / "include" / "ssla_hip.h").read_text()
    defs = {}
    for name, val in re.findall(r"#define\s+(SSLA_\w+)\s+\(?(-?(?:0x)?[0-9A-Fa-f]+)u?\)?", text):
        defs[name] = int(val, 0)
    for name in ("SSLA_OK", "SSLA_ERR_ARG", "SSLA_ERR_HIP", "SSLA_ERR_IO", "SSLA_ERR_FORMAT",
                 "SSLA_ERR_STATE"):
        assert defs[name] == getattr(abi, name), name
    assert defs["SSLA_DRAIN_PHASES"] == len(abi.DRAIN_PHASES)
    assert defs["SSLA_PRED_BUSY"] == abi.PRED_BUSY
