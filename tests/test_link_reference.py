"""The drop-in boundary at link time (CPU; needs the reference tree and the
built library, skipped where the reference tree is absent).

The reference picks its GPU backend by which object it links: gpu.o or
gpu_metal.o (engine/Makefile:112-120; "model.c only uses the gpu.h API, so
it links fine against either backend", engine/Makefile:122-123).  Here:

- the engine's own objects (engine/Makefile:40-48: cli, main, model,
  inference, gguf, memory, tokenizer), compiled in place from the reference
  sources, link against libornith_hip.so with no gpu.o (oracle/Makefile
  `link`); an unresolved gpu_* symbol fails that link;
- every gpu_* symbol those objects reference is exported by the library;
- every declaration of include/ornith/gpu.h is compatible with the
  reference's engine/src/gpu.h: the compiler sees both in one translation
  unit and refuses any conflicting type;
- the reference's own backend contract tests (t_gpu.c, t_gpu_metal.c) link
  against the library too (tests/test_gpu_backend.py runs them on the GPU).
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SRC = "/root/reference/engine/src"
LIB = os.path.join(ROOT, "ornith-flight_amd", "lib", "libornith_hip.so")
REF = os.path.join(ROOT, "oracle", "_ref")

pytestmark = pytest.mark.skipif(not os.path.isdir(REF_SRC) or not os.path.exists(LIB),
                                reason="needs /root/reference and the built library")


@pytest.fixture(scope="module")
def linked():
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "link"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return r


def symbols(path, *flags):
    out = subprocess.run(["nm", *flags, path], capture_output=True, text=True, check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if ln.strip()}


def test_engine_links_without_a_backend_object(linked):
    for exe in ("ornith_hip", "t_gpu_hip", "t_gpu_metal_hip"):
        assert os.access(os.path.join(REF, exe), os.X_OK), exe
    objs = sorted(os.listdir(os.path.join(REF, "link")))
    assert objs == sorted(f"{m}.o" for m in
                          ("cli", "main", "model", "inference", "gguf", "memory", "tokenizer"))
    # what the engine needs from a backend (the gpu.h functions it calls),
    # and what this library exports
    api = set(gpu_decls(preprocessed(os.path.join(REF_SRC, "gpu.h"))))
    need = set()
    for o in objs:
        need |= {s for s in symbols(os.path.join(REF, "link", o), "-u") if s.startswith("gpu_")}
    have = symbols(LIB, "-D", "--defined-only")
    assert need, "the engine references no gpu_* symbol?"
    assert need <= api, sorted(need - api)
    assert need <= have, sorted(need - have)
    # the engine binary resolves them from the library: none of the gpu.h
    # functions is defined in it (model.c's own gpu_*_wrap helpers are)
    exe_defined = symbols(os.path.join(REF, "ornith_hip"), "--defined-only")
    assert not exe_defined & api, sorted(exe_defined & api)
    needed = subprocess.run(["readelf", "-d", os.path.join(REF, "ornith_hip")],
                            capture_output=True, text=True, check=True).stdout
    assert "libornith_hip.so" in needed


def preprocessed(header):
    return subprocess.run(["gcc", "-E", "-P", "-x", "c", header], capture_output=True, text=True,
                          check=True).stdout


def gpu_decls(text):
    """Function declarations of gpu_* names in preprocessed header text."""
    flat = re.sub(r"\s+", " ", text)
    return {m.group(2): m.group(0).strip() for m in
            re.finditer(r"(?:(?<=[;}])|^)\s*([A-Za-z_][^;{}()]*?)\b(gpu_\w+)\s*\([^;{}]*\)\s*;",
                        flat)}


def test_gpu_h_declarations_match_the_reference(tmp_path):
    ours = gpu_decls(preprocessed(os.path.join(ROOT, "include", "ornith", "gpu.h")))
    ref = gpu_decls(preprocessed(os.path.join(REF_SRC, "gpu.h")))
    assert set(ref) == set(ours), (sorted(set(ref) ^ set(ours)))
    # our declarations after the reference's header: any conflicting
    # return or parameter type is a compile error
    tu = tmp_path / "abi.c"
    body = "\n".join(ours.values())
    tu.write_text('#include "gpu.h"\n' + body + "\n")
    r = subprocess.run(["gcc", "-std=c11", "-fsyntax-only", "-Werror", "-Wall", "-I", REF_SRC,
                        str(tu)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    # and a mismatch would be caught: one parameter type changed
    name, decl = next(iter(sorted(ours.items())))
    bad = re.sub(r"\(", "(int, ", decl, count=1) if "(void)" not in decl else \
        decl.replace("(void)", "(int)")
    tu.write_text('#include "gpu.h"\n' + bad + "\n")
    r = subprocess.run(["gcc", "-std=c11", "-fsyntax-only", "-Werror", "-I", REF_SRC, str(tu)],
                       capture_output=True, text=True)
    assert r.returncode != 0 and "conflicting types" in r.stderr, (name, r.stderr)
