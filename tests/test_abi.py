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
