"""Which device launches are the hip backend's own compute kernels.

The reference tells an operator's kernels from everything else by name
(tilebench/profiling/ncu_kernel_select.py:98-102): its Triton/cuTile kernels
are bare identifiers, while ATen and library kernels are mangled C++ (`void
at::native::...<...>`) and the ROCm runtime's copies are `__amd_rocclr_*`.
The hip backend's kernels are C++ too, so the rule here is the namespace:
every kernel of libtbhip.so lives in `tb::`.  rocprofv3 reports it demangled
(`tb::ntg::nt_gemm<1, 2, 256, 256, 128, 64>`), torch.profiler as the mangled
symbol (`_ZN2tb5w4a1613w4a16_prefillEPKDF16_...`), so names are demangled
(libstdc++'s __cxa_demangle) before they are classified.
"""
from __future__ import annotations

import ctypes
import ctypes.util
import functools
import re

_BACKEND = re.compile(r"^(?:void\s+)?tb::")
#: runtime work that is not an operator kernel (copy/fill engines, blit kernels)
_RUNTIME_MARKERS = ("memcpy", "memset")
_RUNTIME_PREFIXES = ("__amd_rocclr_",)


@functools.lru_cache(maxsize=None)
def _cxa_demangle():
    lib = ctypes.CDLL(ctypes.util.find_library("stdc++") or "libstdc++.so.6")
    fn = lib.__cxa_demangle
    fn.restype = ctypes.c_void_p
    fn.argtypes = [ctypes.c_char_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]
    free = ctypes.CDLL(None).free
    free.argtypes = [ctypes.c_void_p]
    return fn, free


@functools.lru_cache(maxsize=4096)
def demangle(name: str) -> str:
    """The demangled form of an Itanium-mangled symbol (`_Z...`); any other
    name unchanged."""
    if not name or not name.startswith("_Z"):
        return name
    text = _demangle_once(name)
    if text is None and "DF16_" in name:
        # Older demanglers lack `DF16_` (_Float16); `Dh` (half) is the same
        # kind of builtin type, so the rest of the symbol parses unchanged.
        text = _demangle_once(name.replace("DF16_", "Dh"))
        text = re.sub(r"\bhalf\b", "_Float16", text) if text is not None else None
    return name if text is None else text


def _demangle_once(symbol: str):
    fn, free = _cxa_demangle()
    status = ctypes.c_int(0)
    out = fn(symbol.encode(), None, None, ctypes.byref(status))
    if not out:
        return None
    try:
        return ctypes.string_at(out).decode() if status.value == 0 else None
    finally:
        free(out)


def is_backend_kernel(name: str) -> bool:
    """True for a kernel of the hip backend (namespace `tb::`), in any of the
    spellings the profilers use."""
    return bool(name) and bool(_BACKEND.match(demangle(name)))


def is_aux_kernel(name: str) -> bool:
    """True for every other device launch: ATen and library kernels, runtime
    copies and fills, and empty names."""
    if not name:
        return True
    name = demangle(name)
    low = name.lower()
    if name.startswith(_RUNTIME_PREFIXES) or any(m in low for m in _RUNTIME_MARKERS):
        return True
    return not is_backend_kernel(name)


def kernel_stem(name: str) -> str:
    """`void tb::ntg::nt_gemm<1, 2, 256, 256, 128, 64>(unsigned char const*, ...)`
    -> `tb::ntg::nt_gemm<1, 2, 256, 256, 128, 64>`: no `void`, no argument list."""
    s = re.sub(r"^void\s+", "", demangle(name.strip()))
    depth = 0
    for i, ch in enumerate(s):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return s[:i]
    return s


def kernel_filter_regex(names) -> str:
    """A regex selecting these kernels by name for rocprofv3
    `--kernel-include-regex` (applied to counter collection and thread trace,
    not to the kernel trace).  rocprofv3 matches it against the full demangled
    signature (`void tb::ntg::nt_gemm<3, 4, 128, 128, 64, 64>(unsigned char
    const*, ...)`: `void ` only before templates) and does not accept `(?:`
    groups, so the regex uses only what POSIX extended and ECMAScript grammars
    read alike: `^`, plain groups, `|`, `?` and backslash-escaped
    metacharacters.  Start-anchored and, like the reference's filter
    (rocprof_compute.py:83-92), never end-anchored."""
    stems = sorted({kernel_stem(n) for n in (names or []) if is_backend_kernel(n)})
    if not stems:
        raise ValueError("no backend kernel names to select")
    alts = ["(void )?" + regex_escape(s) for s in stems]
    # rocprofv3's demangler leaves symbols it cannot read (`DF16_`, _Float16)
    # mangled, so each kernel is also selected by its mangled name's prefix.
    alts += [m for m in (mangled_prefix_regex(s) for s in stems) if m]
    return "^(" + "|".join(alts) + ")"


def _split_scope(stem: str) -> list[str]:
    parts, depth, cur = [], 0, ""
    i = 0
    while i < len(stem):
        ch = stem[i]
        depth += (ch == "<") - (ch == ">")
        if depth == 0 and stem.startswith("::", i):
            parts.append(cur)
            cur, i = "", i + 2
            continue
        cur += ch
        i += 1
    return parts + [cur]


def mangled_prefix_regex(stem: str):
    """The Itanium-mangled prefix of a kernel stem as a regex, e.g.
    `tb::ntg::nt_gemm<3, 4>` -> `_ZN2tb3ntg7nt_gemmIL[a-z]+3EL[a-z]+4EEE`
    (integer template arguments of any integer type, `false` / `true` as
    `Lb0E` / `Lb1E`); None when a template argument is anything else."""
    out = "_ZN"
    for comp in _split_scope(stem):
        name, _, targs = comp.partition("<")
        if not re.fullmatch(r"[A-Za-z_][A-Za-z0-9_]*", name):
            return None
        out += f"{len(name)}{name}"
        if targs:
            args = [a.strip() for a in targs.rstrip(">").split(",")]
            parts = []
            for a in args:
                if a in ("false", "true"):
                    parts.append("Lb" + ("1" if a == "true" else "0") + "E")
                elif re.fullmatch(r"-?[0-9]+", a):
                    parts.append("L[a-z]+" + ("n" + a[1:] if a.startswith("-") else a) + "E")
                else:
                    return None
            out += "I" + "".join(parts) + "E"
    return out + "E"


_META = set("\\^$.|?*+()[]{}")


def regex_escape(text: str) -> str:
    """Backslash-escape the metacharacters shared by POSIX extended and
    ECMAScript regexes and nothing else (Python's re.escape also escapes
    spaces, which those grammars need not read as a plain space)."""
    return "".join("\\" + c if c in _META else c for c in text)
