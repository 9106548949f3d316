"""CPU checks that the reference's Go packages can bind this library through cgo.

tests/golden/cgo_abi.json lists every C function that a non-test file of gpu/matrix,
gpu/optimizer or tensor calls, with the prototype internal/cgo/metal_bridge.h declares for it
(written by tests/golden/make_cgo_abi.py). cgo needs each name declared in the preamble's
header with a compatible type, and the final link needs each one exported. The tests here:

* compile a C file that includes include/gonngpu.h and assigns every listed function to a
  pointer of the reference prototype's type (gcc -Werror: a declaration missing from the
  header, or a different parameter or return type, fails), checks the struct fields the Go
  code reads, links it against libgonngpu.so (an export missing from the library fails the
  link) and runs it (the library loads and resolves);
* check that every entry reported as "not provided" returns -1 with that message and does no
  device work;
* where the reference checkout is present (the build container), regenerate the list from
  the Go sources and compile the same pointer assignments against the reference's own
  header, so the committed list is complete and its prototypes are the reference's.
"""
import ctypes
import json
import os
import subprocess
import sys
import tempfile

import pytest

import gonngpu as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ABI = os.path.join(ROOT, "tests", "golden", "cgo_abi.json")
REF = "/root/reference"
REF_HEADER = os.path.join(REF, "internal", "cgo", "metal_bridge.h")

# Part 3 entries with a device implementation (tested on the GPU in test_compat_gpu.py).
IMPLEMENTED_PART3 = {
    "perform_mps_matrix_add", "perform_mps_matrix_add_broadcast", "perform_mps_matrix_subtract",
    "perform_mps_matrix_element_multiply", "perform_mps_matrix_element_divide", "perform_mps_matrix_scalar_add",
    "perform_mps_matrix_scalar_multiply", "getGPUMemoryUsage",
} | {f"perform_activation_{a}_backward" for a in
     ("relu", "sigmoid", "tanh", "leaky_relu", "elu", "swish", "gelu", "softmax_1d", "softmax_2d")}


def abi():
    with open(ABI) as f:
        return json.load(f)


def pointer_decl(fn):
    params = ", ".join(t for t, _ in fn["params"]) or "void"
    return f"{fn['ret']} (*const p_{fn['name']})({params}) = {fn['name']};"


def field_checks(types):
    lines = []
    for name, t in sorted(types.items()):
        for ftype, fname in t.get("fields", []):
            lines.append(f"_Static_assert(__builtin_types_compatible_p(__typeof__((({name} *)0)->{fname}), {ftype}), "
                         f"\"{name}.{fname}\");")
    return lines


def c_source(data, header):
    fns = data["functions"]
    body = [f'#include "{header}"', "#include <stdio.h>", ""]
    body += [pointer_decl(f) for f in fns]
    body += [""] + field_checks(data["types"]) + [""]
    body.append("int main(void) {")
    body.append("  const void *volatile keep[] = {" + ", ".join(f"(const void *)p_{f['name']}" for f in fns) + "};")
    body.append(f'  printf("%d\\n", (int)(sizeof keep / sizeof keep[0]));')
    body.append("  return 0;")
    body.append("}")
    return "\n".join(body) + "\n"


def gcc(args, cwd):
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-Wno-unused-variable"] + args, cwd=cwd,
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]


def test_list_covers_the_hot_path_and_is_consistent():
    data = abi()
    names = [f["name"] for f in data["functions"]]
    assert len(names) == len(set(names))
    # the matmul path's own entry points are on the list
    for n in ("perform_mps_matrix_multiplication", "perform_mps_matrix_transpose", "perform_sparse_dense_matmul",
              "perform_sparse_matvec", "perform_fused_linear_activation", "perform_optimized_gemm",
              "create_gpu_buffer", "retrieve_gpu_buffer_data", "release_gpu_buffer", "free_c_error_message"):
        assert n in names
    for f in data["functions"]:
        assert f["go_calls"] and f["header_line"] > 0


def test_header_declares_and_library_exports_every_go_called_function():
    data = abi()
    lib_dir = os.path.dirname(G.LIB_PATH)
    if not os.path.exists(G.LIB_PATH):
        pytest.skip("libgonngpu.so is not built")
    with tempfile.TemporaryDirectory() as d:
        with open(os.path.join(d, "link.c"), "w") as f:
            f.write(c_source(data, os.path.join(ROOT, "include", "gonngpu.h")))
        gcc(["link.c", "-o", "link", f"-L{lib_dir}", "-lgonngpu", f"-Wl,-rpath,{lib_dir}", "-Wl,--no-undefined"], d)
        r = subprocess.run([os.path.join(d, "link")], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        assert int(r.stdout.strip()) == len(data["functions"])


def test_header_matches_reference_header_on_every_listed_prototype():
    if not os.path.exists(REF_HEADER):
        pytest.skip("reference checkout not present")
    data = abi()
    with tempfile.TemporaryDirectory() as d:
        with open(os.path.join(d, "ref.c"), "w") as f:
            f.write(c_source(data, REF_HEADER))
        gcc(["-fsyntax-only", "ref.c"], d)


def test_list_is_what_the_reference_go_code_calls():
    if not os.path.exists(REF_HEADER):
        pytest.skip("reference checkout not present")
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    try:
        import make_cgo_abi as M
    finally:
        sys.path.pop(0)
    protos, typedefs = M.parse_header(REF_HEADER)
    uses = M.scan_go(REF)
    called = {n for n in uses if n not in M.NOT_BRIDGE and n in protos}
    data = abi()
    assert called == {f["name"] for f in data["functions"]}
    for f in data["functions"]:
        assert f["ret"] == protos[f["name"]]["ret"] and f["params"] == protos[f["name"]]["params"], f["name"]
    unknown = {n for n in uses if n not in M.NOT_BRIDGE and n not in protos and n not in typedefs}
    assert not unknown, unknown


def _c_arg(ctype):
    if ctype == "float":
        return ctypes.c_float(0.0)
    if ctype in ("long", "int", "unsigned int"):
        return ctypes.c_long(0) if ctype == "long" else ctypes.c_int(0)
    return ctypes.c_void_p(None)  # pointers and opaque handles


def test_not_provided_entries_report_minus_one_with_a_message():
    """Every int-returning entry outside the implemented set returns -1 and names itself;
    called with NULL / zero arguments, it must touch none of them."""
    data = abi()
    lib = G.load()
    bound = set(G.SIGNATURES)
    checked = 0
    for f in data["functions"]:
        name = f["name"]
        if name in bound or name in IMPLEMENTED_PART3 or f["ret"] != "int":
            continue
        err_idx = [i for i, (t, _) in enumerate(f["params"]) if t == "CError*"]
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        args = [_c_arg(t) for t, _ in f["params"]]
        err = G.CError()
        if err_idx:
            args[err_idx[0]] = ctypes.byref(err)
        fn.argtypes = None
        rc = fn(*args)
        assert rc == -1, name
        if err_idx:
            msg = ctypes.string_at(err.message).decode()
            lib.free_c_error_message(err.message)
            assert msg == f"{name}: not provided by the go-nngpu MI355X GEMM/SpMM backend"
        checked += 1
    assert checked >= 80


def test_pointer_and_void_entries_are_inert():
    lib = G.load()
    for name in ("createCommandQueue", "createMetalEvent", "allocateSharedMemory"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_void_p
        assert fn(None) is None
    fn = lib.getGPUCounters
    vals = (ctypes.c_float * 3)(1.0, 2.0, 3.0)
    fn.argtypes = [ctypes.c_void_p]
    fn(ctypes.cast(vals, ctypes.c_void_p))
    assert list(vals) == [0.0, 0.0, 0.0]
    err = G.CError()
    fn = lib.memoryMapFile
    fn.restype = ctypes.c_void_p
    assert fn(b"/nonexistent", None, ctypes.byref(err)) is None
    assert b"memoryMapFile: not provided" in ctypes.string_at(err.message)
    lib.free_c_error_message(err.message)


CGO_PSEUDO = {"CString", "GoString", "GoBytes", "GoStringN", "CBytes", "int", "long", "float", "double", "bool", "uint",
              "size_t", "void", "char", "uchar", "ulong", "schar", "short", "ushort", "longlong", "ulonglong"}


def cgo_preamble(text):
    """The cgo preamble of a Go file: the comment right above `import "C"` (a /* */ block or
    consecutive // lines), or None."""
    lines = text.split("\n")
    idx = next((i for i, l in enumerate(lines) if l.strip() == 'import "C"'), None)
    if idx is None:
        return None
    j = idx - 1
    if lines[j].strip().endswith("*/"):
        k = j
        while "/*" not in lines[k]:
            k -= 1
        block = "\n".join(lines[k:j + 1])
        return block[block.index("/*") + 2:block.rindex("*/")]
    out = []
    while j >= 0 and lines[j].lstrip().startswith("//"):
        out.append(lines[j].lstrip()[2:])
        j -= 1
    return "\n".join(reversed(out))


def test_integration_script_resolves_every_cgo_name_of_every_go_file():
    """go-nngpu_amd/integrate_go.sh applied to a copy of the reference's Go packages: then no
    macOS-only directive is left, and for every Go file with a cgo preamble, that preamble
    (which includes the replaced internal/cgo/metal_bridge.h) declares every C name the file
    uses, which is what cgo checks first ("could not determine kind of name for C.x").
    Each preamble is compiled by gcc with a reference to each such name."""
    import re
    import shutil

    if not os.path.exists(REF_HEADER):
        pytest.skip("reference checkout not present")
    with tempfile.TemporaryDirectory() as d:
        for sub in ("gpu", "tensor", "internal"):
            shutil.copytree(os.path.join(REF, sub), os.path.join(d, sub))
        r = subprocess.run(["sh", os.path.join(ROOT, "go-nngpu_amd", "integrate_go.sh"), d, ROOT],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
        assert not [f for f in os.listdir(os.path.join(d, "internal", "cgo")) if f.endswith((".m", ".metal"))]
        fused = open(os.path.join(d, "gpu", "matrix", "fused-operations.go")).read()
        assert "activationType := C.int(ReLU)" in fused and "C.int(OpReLU)" not in fused
        checked = 0
        for sub in ("gpu", "tensor", "internal"):
            for root, _, files in os.walk(os.path.join(d, sub)):
                for fn in sorted(files):
                    if not fn.endswith(".go") or fn.endswith("_test.go"):
                        continue
                    path = os.path.join(root, fn)
                    text = open(path).read()
                    pre = cgo_preamble(text)
                    if pre is None:
                        continue
                    directives = [l.strip() for l in pre.split("\n") if l.strip().startswith("#cgo")]
                    assert directives and all("-lgonngpu" in l and "-framework" not in l for l in directives), \
                        (path, directives)
                    code = "\n".join(l for l in text.split("\n") if not l.lstrip().startswith("//"))
                    names = sorted(set(re.findall(r"\bC\.([A-Za-z_]\w*)", code)) - CGO_PSEUDO)
                    refs = []
                    for n in names:
                        if n in ("GPUPtr", "DevicePtr", "CError", "GPUCounters", "KernelCompileOptions"):
                            refs.append(f"  (void)sizeof({n});")
                        else:
                            refs.append(f"  (void)&{n};")
                    src = "\n".join(l for l in pre.split("\n") if not l.strip().startswith("#cgo"))
                    src += "\nvoid cgo_name_check(void) {\n" + "\n".join(refs) + "\n}\n"
                    cfile = os.path.join(root, "_cgo_check_" + fn[:-3] + ".c")
                    with open(cfile, "w") as f:
                        f.write(src)
                    r = subprocess.run(["gcc", "-std=gnu11", "-fsyntax-only", "-Werror", cfile], capture_output=True,
                                       text=True)
                    assert r.returncode == 0, (path, r.stderr[-3000:])
                    checked += 1
        assert checked == 35
