"""Host-side checks that need no GPU: the C-ABI library loads and exports every
entry point include/lisa_hip.h declares; the speculative acceptance and
drafter-reconcile golden tables of the reference (src/speculative/mod.rs:
458-547) through the product's C ABI; the hybrid layer schedule
(src/model/mod.rs:29-39)."""
import re
from pathlib import Path

import pytest

from _lisa import load_oracle, load_pkg

ROOT = Path(__file__).resolve().parents[1]


def declared_entry_points():
    text = (ROOT / "include" / "lisa_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(lisa_\w+)\s*\(", text, re.M)
    return sorted(set(names))


def test_c_abi_exports_every_declared_symbol():
    pkg = load_pkg()
    lib = pkg.lib()  # fails loudly if liblisa_hip.so or the kernel module is missing
    names = declared_entry_points()
    assert len(names) >= 50
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_kernel_module_is_built_for_gfx950():
    pkg = load_pkg()
    blob = Path(pkg.HSACO_PATH).read_bytes()
    # hipcc --genco writes a clang offload bundle holding one gfx950 code object
    assert blob.startswith(b"__CLANG_OFFLOAD_BUNDLE__") or blob[:4] == b"\x7fELF"
    assert b"amdgcn-amd-amdhsa--gfx950" in blob or b"gfx950" in blob
    for name in (b"lisa_qmv_k5120_m1_resnorm", b"lisa_qmv_k17408_m1_x", b"lisa_gdn_recurrence_m1",
                 b"lisa_attn_partial_m1", b"lisa_attn_merge_m1", b"lisa_step_finalize"):
        assert name in blob


@pytest.mark.parametrize("drafts,target,accepted,emitted,trim", [
    ([10, 11], [20, 21, 22], 0, [20], 2),        # rejects_first_draft
    ([10, 11], [10, 21, 22], 1, [10, 21], 1),    # accepts_one_draft
    ([10, 11], [10, 11, 22], 2, [10, 11, 22], 0),  # accepts_all_drafts_and_bonus
])
def test_accept_greedy_golden(drafts, target, accepted, emitted, trim):
    r = load_pkg().accept_greedy(drafts, target)
    assert (r.accepted_drafts, list(r.emitted), r.target_trim) == (accepted, emitted, trim)


@pytest.mark.parametrize("args,trim,replay", [
    ((2, 2, 0), 2, [("replacement",)]),          # reconciles_first_round_transitions
    ((2, 2, 1), 1, [("replacement",)]),
    ((2, 2, 2), 0, [("replacement",)]),
    ((2, 1, 0), 1, [("replacement",)]),          # reconciles_seeded_round_transitions
    ((2, 1, 1), 0, [("replacement",)]),
    ((2, 1, 2), 0, [("draft", 1), ("replacement",)]),
])
def test_mtp_reconcile_plan_golden(args, trim, replay):
    assert load_pkg().mtp_reconcile_plan(*args) == (trim, replay)


def test_accept_greedy_rejects_bad_lengths():
    with pytest.raises(ValueError):
        load_pkg().accept_greedy([1, 2], [1, 2])


def test_layer_schedule():
    """64 layers: every fourth is full attention, 16 in all (src/model/mod.rs:29-39)."""
    orc = load_oracle()
    attn = [i for i in range(64) if orc.layer_is_attention(i)]
    assert len(attn) == 16
    assert attn == list(range(3, 64, 4))


def test_cond_offset_mapping():
    """The Rust shim passes the reference's (buffer, byte offset) conditioning
    (speculative/mod.rs:141-183) through lisa_mtp_forward_device; the library
    maps it onto (cond_source, cond_row): target hidden row r at
    hidden_offset(r), the drafter's own hidden at normalized_offset()."""
    pkg = load_pkg()
    for row in range(3):
        assert pkg.resolve_cond(True, pkg.hidden_offset(row)) == (0, row)
    assert pkg.hidden_offset(1) - pkg.hidden_offset(0) == 5120 * 2
    assert pkg.resolve_cond(False, pkg.normalized_offset()) == (1, 0)
    for bad in (pkg.hidden_offset(3), pkg.hidden_offset(1) + 2, 7):
        with pytest.raises(pkg.LisaError) as err:
            pkg.resolve_cond(True, bad)
        assert err.value.code == -1
    with pytest.raises(pkg.LisaError):
        pkg.resolve_cond(False, pkg.normalized_offset() + 16)
