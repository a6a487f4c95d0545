"""The SBCL binding (ex-nihilo_amd/lisp/hip-dit.lisp, hip-vae.lisp, hip-vision.lisp, hip-encoder.lisp)
against the C ABI, without
SBCL (neither this image nor the GPU host has it): every define-alien-routine names a function
that include/exn_hip.h declares, with its arity and, argument by argument, a Lisp alien type
that passes the C type (int, 64-bit integers, double, pointers, C strings); and the backend trio
keeps the reference's lambda lists (src/cuda-dit.lisp:52,137,99; src/cuda-vae.lisp:15,94,138,28;
src/cuda-vision.lisp:15,34,103; src/encoder.lisp:41,50,69,143)."""
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LISP = os.path.join(REPO, "ex-nihilo_amd", "lisp")
HEADER = os.path.join(REPO, "include", "exn_hip.h")
FILES = ("hip-dit.lisp", "hip-vae.lisp", "hip-vision.lisp", "hip-encoder.lisp")


def prototypes():
    """name -> (return type, [parameter types]) from the header."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(int|const char\*)\s+(exn_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.M | re.S):
        ret, name, params = m.group(1), m.group(2), " ".join(m.group(3).split())
        types = []
        if params and params != "void":
            for p in params.split(","):
                p = p.strip()
                t = re.sub(r"\s*\b\w+$", "", p) if not p.endswith("*") else p   # drop the parameter name
                types.append(t.replace(" *", "*").strip())
        out[name] = (ret, types)
    return out


def sexprs(text):
    """The top-level forms of a Lisp file as nested lists of atoms (strings)."""
    # strings first (a ';' inside a docstring starts no comment), then comments, parens, atoms
    tokens = [t for t in re.findall(r'"(?:\\.|[^"])*"|;[^\n]*|[()]|[^\s()]+', text) if not t.startswith(";")]
    stack, top = [], []
    for t in tokens:
        if t == "(":
            stack.append([])
        elif t == ")":
            f = stack.pop()
            (stack[-1] if stack else top).append(f)
        else:
            (stack[-1] if stack else top).append(t)
    assert not stack, "unbalanced parentheses"
    return top


def forms(name):
    return sexprs(open(os.path.join(LISP, name)).read())


def alien_routines():
    out = {}
    for f in FILES:
        for form in forms(f):
            if isinstance(form, list) and form and form[0] == "sb-alien:define-alien-routine":
                cname = form[1][0].strip('"')
                out[cname] = (form[2], [a[1] for a in form[3:]])
    return out


def passes(lisp_type, c_type):
    """Whether the alien type carries the C type across the call."""
    if isinstance(lisp_type, list):
        kind, bits = lisp_type[0], int(lisp_type[1])
        return bits == 64 and ((kind == "sb-alien:signed" and c_type == "int64_t") or
                               (kind == "sb-alien:unsigned" and c_type in ("uint64_t", "size_t")))
    if lisp_type == "sb-alien:int":
        return c_type == "int"
    if lisp_type == "sb-alien:double":
        return c_type == "double"
    if lisp_type == "sb-alien:float":
        return c_type == "float"
    if lisp_type == "sb-alien:c-string":
        return c_type == "const char*"
    if lisp_type == "sb-sys:system-area-pointer":
        return c_type.endswith("*")
    return False


def test_every_alien_routine_matches_the_header():
    protos = prototypes()
    routines = alien_routines()
    assert len(routines) >= 10
    for cname, (ret, args) in routines.items():
        assert cname in protos, cname
        cret, cargs = protos[cname]
        assert len(args) == len(cargs), (cname, args, cargs)
        assert passes(ret, "const char*" if cret == "const char*" else "int"), (cname, ret, cret)
        for i, (la, ca) in enumerate(zip(args, cargs)):
            assert passes(la, ca), (cname, i, la, ca)


def test_the_trio_keeps_the_reference_lambda_lists():
    defs = {}
    for f in FILES:
        for form in forms(f):
            if isinstance(form, list) and form and form[0] == "defun":
                defs[form[1]] = form[2]
    assert defs["upload-dit"] == ["path", "&key", ["device", "0"]]
    assert defs["dit-velocity"] == ["d", "context", "p", "latent", "h", "w", "sigma", "&key", ["prefix-key", "nil"],
                                    "ref"]
    assert defs["dit-release"] == ["d"]
    assert defs["upload-vae"] == ["path", "&key", ["device", "0"]]
    assert defs["vae-decode"] == ["v", "latent", "h", "w"]
    assert defs["vae-encode"] == ["v", "px", "h", "w"]   # src/cuda-vae.lisp:138
    assert defs["vae-release"] == ["v"]
    assert defs["load-vision"] == ["path", "&key", ["device", "1"]]
    assert defs["vision-encode"] == ["v", "px", "h", "w"]
    assert defs["vision-release"] == ["v"]
    assert defs["load-encoder"] == ["path", "&key", "device", ["threads", ["il::default-thread-count"]]]
    # the encoder's compute only (src/encoder.lisp:50,69,143); encode-prompt and encode-edit-prompt
    # stay the reference's own (:55-141), which load before and call these
    assert defs["encoder-gpu-p"] == ["model"]
    assert defs["call-with-picture-rows"] == ["model", "merged", "deep", "d", "rows-in", "fn"]
    assert defs["encoder-states"] == ["model", "ids", "&key", "rope"]
    assert "encode-prompt" not in defs and "encode-edit-prompt" not in defs


def test_the_header_parse_sees_the_trio():
    p = prototypes()
    assert p["exn_dit_velocity"][1] == ["exn_dit*", "const float*", "int", "const float*", "int", "int", "double",
                                        "uint64_t", "int", "const float*", "int", "int", "float*"]
    assert p["exn_last_error"] == ("const char*", [])


@pytest.mark.parametrize("name", FILES)
def test_files_parse_and_stay_in_the_package(name):
    fs = forms(name)
    assert fs[0] == ["in-package", "#:ex-nihilo"]


def flatten(form):
    if isinstance(form, list):
        for f in form:
            yield from flatten(f)
    else:
        yield form


def test_diagnostics_mirror_the_reference():
    """dit-velocity turns the library's numbers on as the reference's switches ask: *dit-trace*
    (src/metal-dit.lisp:114-117, printed per layer as its trace-max prints) through exn_dit_stats,
    and EXN_PROFILE (src/tenant.lisp:53-62) through exn_dit_profile, its classes' seconds added
    to illatio's *gpu-profile* table that tenant-run reports."""
    fs = {f[1]: f for f in forms("hip-dit.lisp") if isinstance(f, list) and len(f) > 1 and f[0] in ("defun", "defvar")}
    assert "*dit-trace*" in fs
    vel = list(flatten(fs["dit-velocity"]))
    for atom in ('"EXN_PROFILE"', "il::*gpu-profile*", "%exn-dit-stats", "%exn-dit-profile", "*dit-trace*",
                 "print-dit-trace", "add-gpu-profile"):
        assert atom in vel or "'" + atom in vel, atom
    trace = list(flatten(fs["print-dit-trace"]))
    assert "%exn-dit-stats-read" in trace and '"x"' in trace and '"att"' in trace and '"ff"' in trace
    prof = list(flatten(fs["add-gpu-profile"]))
    assert "%exn-dit-profile-read" in prof and "gethash" in prof
