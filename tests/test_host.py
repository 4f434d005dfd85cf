"""Host-side logic and the C ABI library (no GPU compute)."""
import ctypes
import json
import re
from pathlib import Path

import numpy as np
import pytest

from conftest import ROOT, load_golden


def _declared_functions() -> list[str]:
    names = []
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(wc_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    from woodcock_amd import _lib

    declared = _declared_functions()
    assert "wc_kv_compact" in declared and "wc_verify_chain_greedy" in declared
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared if not hasattr(handle, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert sorted(_lib.exported_symbols()) == declared, "ctypes signatures must cover exactly the header"


def test_ctypes_structs_match_the_header(tmp_path):
    """Sizes and field offsets of the ctypes mirrors equal the C header's (gcc
    compiles a probe against include/woodcock_hip.h)."""
    import shutil
    import subprocess

    from woodcock_amd import _lib

    if not shutil.which("gcc"):
        pytest.skip("no C compiler")
    mirrors = {"wc_drafter_dims": _lib.DrafterDims, "wc_layer_weights": _lib.LayerWeights,
               "wc_drafter_weights": _lib.DrafterWeights, "wc_gumbel": _lib.Gumbel, "wc_uniforms": _lib.Uniforms}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "woodcock_hip.h"', "int main(void) {"]
    for cname, py in mirrors.items():
        lines.append(f'  printf("{cname} %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'  printf("{cname}.{f} %zu\\n", offsetof({cname}, {f}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                          check=True).stdout.splitlines())
    for cname, py in mirrors.items():
        assert int(got[cname]) == ctypes.sizeof(py), cname
        for f, _ in py._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(py, f).offset, f"{cname}.{f}"


def test_library_loads_and_reports_abi():
    from woodcock_amd import _lib

    L = _lib.lib()
    assert L.wc_version() == _lib.ABI_VERSION
    assert L.wc_workspace_bytes() >= 8 * _lib.WC_MAX_NODES


def test_verdict_layout_matches_header():
    from woodcock_amd import _lib

    assert _lib.VERDICT_BYTES == 4 * (8 + 2 * (_lib.WC_MAX_NODES + 1))
    text = (ROOT / "include" / "woodcock_hip.h").read_text()
    assert f"#define WC_MAX_NODES {_lib.WC_MAX_NODES}" in text
    assert f"#define WC_ABI_VERSION {_lib.ABI_VERSION}" in text


def test_host_errors_before_any_device_call():
    """Argument errors surface as ValueError from the library's own checks."""
    from woodcock_amd import _lib

    L = _lib.lib()
    rc = L.wc_verify_chain_greedy(None, 5, 10, 10, None, None, None, None)
    assert rc == _lib.WC_E_INVALID and b"NULL" in L.wc_last_error()
    rc = L.wc_kv_compact(None, None, 0, 1, 1, 4, None, None, None, 1, None, None, None)
    assert rc == _lib.WC_E_INVALID
    with pytest.raises(ValueError):
        _lib.check(rc)


# ------------------------------------------------------------------ config and vocabulary

def test_drafter_config_roundtrip_and_legacy_fields(tmp_path):
    """python/woodcock/drafter.py:51-63 and tests/test_drafter.py:71-85."""
    from woodcock_amd.config import DrafterConfig, tiny_drafter

    cfg = tiny_drafter(window=6)
    p = tmp_path / "config.json"
    cfg.save(p)
    assert DrafterConfig.load(p) == cfg
    d = json.loads(p.read_text())
    d.update(residual="feature", lowrank_rank=0, lowrank_k=128)
    p.write_text(json.dumps(d))
    assert DrafterConfig.load(p) == cfg
    for bad in ({"residual": "token"}, {"lowrank_rank": 128}):
        p.write_text(json.dumps({**d, **bad}))
        with pytest.raises(ValueError):
            DrafterConfig.load(p)


def test_top_ids_known_answers():
    """tests/test_vocab.py:13-22."""
    from woodcock_amd.vocab import top_ids

    counts = np.array([5, 0, 9, 5, 1, 7, 0, 0])
    assert top_ids(counts, 3).tolist() == [0, 2, 5]
    assert top_ids(counts, 3, {6}).tolist() == [2, 5, 6]
    assert top_ids(counts, 2, {2}).tolist() == [2, 5]
    with pytest.raises(ValueError):
        top_ids(counts, 0)
    with pytest.raises(ValueError):
        top_ids(counts, 1, {1, 6})


def test_load_ids(tmp_path):
    from woodcock_amd.vocab import load_ids

    np.savez(tmp_path / "c.npz", counts=np.arange(64), eos=np.array([0]))
    ids = load_ids(f"{tmp_path / 'c.npz'}:4")
    assert ids.tolist() == [0, 61, 62, 63] and ids.dtype == np.int32


def test_tree_mask_known_answer_and_goldens():
    """tests/test_sampling.py:199-205 and reference tree_mask goldens."""
    from woodcock_amd.sampling import DraftTree, tree_attention_mask

    tree = DraftTree(tokens=[0, 1, 2, 4], parents=[-1, 0, 0, 2], depth=[0, 1, 1, 2])
    m = tree_attention_mask(tree, prefix_len=2)
    assert m.shape == (4, 6) and m[:, :2].all()
    assert list(m[3, 2:]) == [True, False, True, True]
    assert list(m[1, 2:]) == [True, True, False, False]
    z = load_golden("verify.npz")
    for c in range(40):
        t = DraftTree(z[f"t{c}.tokens"].tolist(), z[f"t{c}.parents"].tolist(), z[f"t{c}.depth"].tolist())
        np.testing.assert_array_equal(tree_attention_mask(t, int(z[f"t{c}.prefix"])), z[f"t{c}.mask"])
