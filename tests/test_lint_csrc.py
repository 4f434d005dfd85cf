"""Source checks of the HIP kernels (CPU only).

MFMA result reads: on gfx950 the compiler's own wait-state count between a
v_mfma and the first read of its result registers has fallen short (tile
elements read stale, differently from run to run), so every kernel that runs
MFMAs -- directly or through a device helper -- drains them with
``mfma_settle()`` after its MFMA loops.  This test finds every such kernel in
``woodcock_amd/csrc`` and checks that each MFMA site (the builtin, or a call of
a helper containing it) is followed by a ``mfma_settle()`` in the kernel body.
"""
import re
from pathlib import Path

CSRC = Path(__file__).resolve().parents[1] / "woodcock_amd" / "csrc"
MFMA = "__builtin_amdgcn_mfma_"
SETTLE = "mfma_settle()"
ATTR = (r"(?:\s*(?:__launch_bounds__\s*\([^)]*\)|__attribute__\s*\(\((?:[^()]|\([^()]*\))*\)\)|__forceinline__"
        r"|__noinline__|static|inline))*")
DEF = re.compile(r"(__global__|__device__)" + ATTR + r"\s+[^;{}()]*?\b(\w+)\s*\(", re.S)


def _strip_comments(src: str) -> str:
    src = re.sub(r"/\*.*?\*/", lambda m: " " * len(m.group(0)), src, flags=re.S)
    return re.sub(r"//[^\n]*", lambda m: " " * len(m.group(0)), src)


def _functions(src: str):
    """(kind, name, body) of every __global__ / __device__ function definition."""
    out = []
    for m in DEF.finditer(src):
        i = src.find("{", m.end())
        semi = src.find(";", m.end())
        if i < 0 or (0 <= semi < i):
            continue  # a declaration
        depth, j = 0, i
        while j < len(src):
            if src[j] == "{":
                depth += 1
            elif src[j] == "}":
                depth -= 1
                if depth == 0:
                    break
            j += 1
        out.append((m.group(1), m.group(2), src[i:j + 1]))
    return out


def _all_functions():
    funcs = []
    for p in sorted(CSRC.glob("*")):
        if p.suffix in (".h", ".hip"):
            funcs += [(p.name, *f) for f in _functions(_strip_comments(p.read_text()))]
    return funcs


def test_mfma_results_are_settled():
    funcs = _all_functions()
    helpers = {name for _, kind, name, body in funcs if kind == "__device__" and MFMA in body and name != "mfma_settle"}
    kernels = 0
    for fname, kind, name, body in funcs:
        if kind != "__global__":
            continue
        sites = [m.start() for m in re.finditer(re.escape(MFMA), body)]
        for h in helpers:
            sites += [m.start() for m in re.finditer(r"\b" + re.escape(h) + r"\s*<[^;()]*>\s*\(|\b" + re.escape(h) +
                                                     r"\s*\(", body)]
        if not sites:
            continue
        kernels += 1
        settles = [m.start() for m in re.finditer(re.escape(SETTLE), body)]
        for s in sites:
            assert any(t > s for t in settles), f"{fname}: kernel {name} reads MFMA results without mfma_settle()"
    assert kernels >= 5, "the MFMA kernels were not found"  # k_gemvf, k_gemvs, k_mm_stream, k_mm_wave, ...


def test_lint_catches_a_missing_settle():
    """The check itself: a kernel with an MFMA and no settle is flagged."""
    src = ("__device__ void helper(float* a) { a[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, y, z, 0, 0, 0); }\n"
           "__global__ void k_bad(float* a) { helper(a); a[1] = 0; }\n"
           "__global__ void k_good(float* a) { helper(a); mfma_settle(); a[1] = 0; }\n")
    funcs = _functions(src)
    assert [f[1] for f in funcs] == ["helper", "k_bad", "k_good"]
    body = {name: b for _, name, b in funcs}
    assert MFMA in body["helper"] and SETTLE not in body["k_bad"] and SETTLE in body["k_good"]
