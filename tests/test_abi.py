"""The C ABI library loads on the CPU and exports every symbol include/vmi.h
declares; argument validation runs without touching a device."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "vmi.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vmi_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    import vates_amd._lib as L
    if not L.LIB_PATH.exists():
        pytest.fail("libvmi.so is not built (run __graft_entry__.build())")
    return L.load()


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), n


def test_python_binding_covers_header():
    import vates_amd._lib as L
    assert sorted(L.exported_names()) == declared_functions()


def test_version_and_workspace_queries(lib):
    assert lib.vmi_version() == 1
    # at least the per-(distinct slot, token) bf16 activation operands of the down projection,
    # and the fp32 path's activation and output rows per pair
    assert lib.vmi_fused_moe_slots_workspace_bytes(4, 10, 2048, 512) >= (4 * 10 + 1) * 4 * 512 * 2
    assert lib.vmi_fused_moe_slots_workspace_bytes(4, 10, 2048, 512) >= 4 * 10 * (512 + 2048) * 4
    # the whole layer also holds the router logits [T, E]
    assert lib.vmi_moe_layer_workspace_bytes(4, 10, 2048, 512, 512) >= (4 * 10 + 1) * 4 * 512 * 2 + 4 * 512 * 4
    assert lib.vmi_fused_moe_slots_workspace_bytes(0, 10, 2048, 512) == 0


def test_invalid_arguments_rejected_before_any_device_call(lib):
    import vates_amd._lib as L
    q = L.QMat(None, None, None)
    rc = lib.vmi_fused_moe_slots(None, 0, None, None, q, q, q, 0, 10, 2048, 512, 64, 4, 512, None, 0, None, 0, None)
    assert rc == L.VMI_ERR_INVALID
    assert b"T=0" in lib.vmi_last_error()
    rc = lib.vmi_fused_moe_slots(None, 0, None, None, q, q, q, 4, 10, 2048, 512, 32, 4, 512, None, 0, None, 0, None)
    assert rc == L.VMI_ERR_UNSUPPORTED
    rc = lib.vmi_fused_moe_slots(None, 0, None, None, q, q, q, 17, 1, 2048, 512, 64, 4, 512, None, 0, None, 0, None)
    assert rc == L.VMI_ERR_UNSUPPORTED
    rc = lib.vmi_moe_layer(None, None, 4, None, None, None, None, None, 0, None)
    assert rc == L.VMI_ERR_INVALID
    # the prefill tables: two fp16 halves per (row, group) of gate, up and down
    # for every slot and the shared expert, plus a factor per row
    assert lib.vmi_moe_prefill_tables_bytes(2048, 512, 512) >= 513 * (2 * 512 * 32 + 2048 * 8) * 4
    assert lib.vmi_moe_prefill_tables_bytes(2048, 100, 512) == 0
    assert lib.vmi_moe_prefill_tables(None, None, 0, None) == L.VMI_ERR_INVALID
    d = L.MoeLayerDesc()
    d.hidden, d.inter, d.cap, d.bits, d.group = 2048, 512, 512, 4, 64
    rc = lib.vmi_moe_prefill_tables(ctypes.byref(d), None, 0, None)
    assert rc == L.VMI_ERR_INVALID and b"scales" in lib.vmi_last_error()
    rc = lib.vmi_spec_commit(None, None, 4, 1, 2048, 0, None, None, None, None, None, None, None)
    assert rc == L.VMI_ERR_INVALID and b"K=0" in lib.vmi_last_error()
    rc = lib.vmi_spec_commit(None, None, 0, 1, 2048, 3, None, None, None, None, None, None, None)
    assert rc == L.VMI_ERR_INVALID and b"rows=0" in lib.vmi_last_error()
    rc = lib.vmi_spec_commit(None, None, 4, 1, 2048, 3, None, None, None, None, None, None, None)
    assert rc == L.VMI_ERR_INVALID


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    import vates_amd._lib as L
    monkeypatch.setattr(L, "_lib", None)
    monkeypatch.setattr(L, "LIB_PATH", tmp_path / "libvmi.so")
    with pytest.raises(L.VmiError):
        L.load()
