"""The Rust binding (sys1rust_amd/laya-hip) against the C header it binds.

No Rust toolchain is needed: the declarations of src/ffi.rs are parsed and compared, item by
item, with include/sys1hip.h (names, argument order, C types, struct fields, constants), so a
change to the header that the binding does not follow fails here. The binding's own unit tests
(`cargo test -p laya-hip`) run where sys1rust is built.
"""
from __future__ import annotations

import re
from pathlib import Path

import pytest

from sys1rust_amd.backend import DEFAULT_TUNING

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sys1hip.h"
CRATE = ROOT / "sys1rust_amd" / "laya-hip"

# C type -> Rust type, as the binding must spell it.
C_TO_RUST = {
    "int": "c_int",
    "int32_t": "i32",
    "uint32_t": "u32",
    "uint64_t": "u64",
    "size_t": "usize",
    "float": "f32",
    "const char*": "*const c_char",
    "const void*": "*const c_void",
    "const uint32_t*": "*const u32",
    "const uint64_t*": "*const u64",
    "float*": "*mut f32",
    "s1_model*": "*mut S1Model",
    "const s1_model*": "*const S1Model",
    "s1_model**": "*mut *mut S1Model",
    "const s1_tensor*": "*const S1Tensor",
}


def _strip_c_comments(s: str) -> str:
    s = re.sub(r"/\*.*?\*/", " ", s, flags=re.S)
    return re.sub(r"//[^\n]*", " ", s)


def _norm_c_type(t: str) -> str:
    t = re.sub(r"\s*\*\s*", "*", " ".join(t.split()))
    return t


def c_functions() -> dict[str, tuple[str, list[tuple[str, str]]]]:
    text = _strip_c_comments(HEADER.read_text())
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(s1\w*)\s*\(([^)]*)\)\s*;", text):
        ret, name, params = _norm_c_type(m.group(1)), m.group(2), m.group(3).strip()
        args = []
        if params and params != "void":
            for p in params.split(","):
                p = " ".join(p.split())
                pm = re.match(r"(.*?)(\w+)$", p)
                args.append((pm.group(2), _norm_c_type(pm.group(1))))
        out[name] = (ret, args)
    return out


def c_defines() -> dict[str, int]:
    return {k: int(v) for k, v in re.findall(r"#define\s+(S1_\w+)\s+(-?\d+)", HEADER.read_text())}


def rust_functions() -> dict[str, tuple[str, list[tuple[str, str]]]]:
    text = (CRATE / "src" / "ffi.rs").read_text()
    block = re.search(r'extern "C"\s*\{(.*?)\n\}', text, flags=re.S).group(1)
    out = {}
    for m in re.finditer(r"pub fn (\w+)\s*\(([^)]*)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        name, params, ret = m.group(1), m.group(2), (m.group(3) or "").strip()
        args = []
        for p in params.split(","):
            p = " ".join(p.split())
            if p:
                n, t = p.split(":", 1)
                args.append((n.strip(), t.strip()))
        out[name] = (ret, args)
    return out


def test_every_declared_function_matches_the_header():
    c, r = c_functions(), rust_functions()
    assert r, "no extern block parsed"
    for name, (ret, args) in r.items():
        assert name in c, f"{name} is not declared in include/sys1hip.h"
        cret, cargs = c[name]
        want_ret = "" if cret == "void" else C_TO_RUST[cret]
        assert ret == want_ret, (name, ret, cret)
        assert [n for n, _ in args] == [n for n, _ in cargs], (name, args, cargs)
        for (n, t), (_, ct) in zip(args, cargs):
            assert t == C_TO_RUST[ct], (name, n, t, ct)


def test_the_binding_declares_the_whole_model_api():
    """Every model-level entry point (the Backend surface, not the harness or kernel ones)."""
    model_api = {"s1_model_create", "s1_model_create_from_bytes", "s1_model_create_from_tensors",
                 "s1_check_settings", "s1_forward", "s1_encoder_hidden", "s1_padded_len", "s1_name",
                 "s1_active_kernels", "s1_warmup", "s1_last_error", "s1_model_destroy"}
    assert model_api <= set(c_functions())
    assert model_api <= set(rust_functions())


def test_constants_and_tensor_struct_match():
    d = c_defines()
    text = (CRATE / "src" / "ffi.rs").read_text()
    consts = {k: int(v) for k, v in re.findall(r"pub const (S1_\w+): \w+ = (-?\d+);", text)}
    assert consts, "no constants parsed"
    for k, v in consts.items():
        assert d[k] == v, (k, v, d.get(k))
    assert {k for k in d if k.startswith(("S1_ERR", "S1_DTYPE"))} <= set(consts)
    header = _strip_c_comments(HEADER.read_text())
    cfields = re.search(r"typedef struct s1_tensor \{(.*?)\} s1_tensor;", header, flags=re.S).group(1)
    cf = [(m.group(2), _norm_c_type(m.group(1))) for m in re.finditer(r"([\w\s\*]+?)(\w+);", cfields)]
    rfields = re.search(r"pub struct S1Tensor \{(.*?)\}", text, flags=re.S).group(1)
    rf = re.findall(r"pub (\w+): ([^,]+),", rfields)
    assert [n for n, _ in rf] == [n for n, _ in cf]
    for (n, t), (_, ct) in zip(rf, cf):
        assert t.strip() == C_TO_RUST[ct], (n, t, ct)


def test_lib_uses_only_declared_functions_and_exports_laya_mlx_names():
    lib = (CRATE / "src" / "lib.rs").read_text()
    used = set(re.findall(r"\b(s1_\w+)\s*\(", lib))
    assert used <= set(rust_functions()), used - set(rust_functions())
    # The names sys1rust and sys1-bench call on laya_mlx, under this crate's spelling.
    for item in ["pub fn make_backend(", "pub fn factory(", "pub fn check_settings(",
                 "pub const HIP_ENV_DEFAULTS", "pub fn set_hip_env_defaults("]:
        assert item in lib, item
    # The production settings string in the crate's own test is the one the runtime ships.
    assert DEFAULT_TUNING in lib


def _call_args(text: str, start: int) -> list[str]:
    """The top-level comma-separated arguments of the call whose '(' is at text[start]."""
    depth, cur, args = 0, [], []
    for ch in text[start:]:
        if ch in "([{":
            depth += 1
            if depth == 1:
                continue
        elif ch in ")]}":
            depth -= 1
            if depth == 0:
                break
        if depth == 1 and ch == ",":
            args.append("".join(cur).strip())
            cur = []
        else:
            cur.append(ch)
    last = "".join(cur).strip()
    if last:
        args.append(last)
    return args


def test_lib_calls_pass_the_declared_argument_counts():
    """Every call of a C function in src/lib.rs passes as many arguments as src/ffi.rs declares
    (and the header takes), counted at the top level of the call's parentheses."""
    decl = rust_functions()
    lib = (CRATE / "src" / "lib.rs").read_text()
    calls = 0
    for m in re.finditer(r"\b(s1_\w+)\s*\(", lib):
        name = m.group(1)
        if lib[max(0, m.start() - 7): m.start()].endswith("fn "):
            continue  # a definition, not a call
        args = _call_args(lib, m.end() - 1)
        assert len(args) == len(decl[name][1]), (name, args, decl[name][1])
        calls += 1
    assert calls >= 10, calls


@pytest.mark.parametrize("needle", ["Device::Cpu", "library_settings(&opts.settings(), opts.f32)", "\"dtype=f32\"",
                                    "w.view()?", "s1_model_create_from_tensors"])
def test_lib_refuses_cpu_maps_f32_and_binds_through_the_view(needle):
    assert needle in (CRATE / "src" / "lib.rs").read_text()
