"""Writes tests/golden/cgo_abi.json: every C function the reference's Go packages call
through cgo, with the prototype the reference header declares for it (interface data).

Runs only where the reference checkout is present (this build container); the JSON it
writes is committed and is what tests/test_cgo_link.py checks the library against.

Sources scanned (text only, nothing is run or imported):
  gpu/matrix/*.go, gpu/optimizer/*.go, tensor/*.go   `C.<name>` references, excluding
                                                      _test.go files (go build skips them)
  internal/cgo/metal_bridge.h                         prototypes and the typedefs the Go
                                                      code names (C.GPUCounters, ...)
Usage: python tests/golden/make_cgo_abi.py [/root/reference]
"""
import glob
import json
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PACKAGES = ("gpu/matrix", "gpu/optimizer", "tensor")
# C names the Go files use that are not the bridge's: cgo pseudo-functions, libc, C types.
NOT_BRIDGE = {"CString", "GoString", "GoBytes", "free", "malloc", "memcpy", "int", "long", "float", "double",
              "bool", "uint", "size_t", "void", "char", "uchar", "ulong"}


def strip_comments(text):
    text = re.sub(r"/\*.*?\*/", lambda m: "\n" * m.group(0).count("\n"), text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def parse_header(path):
    raw = open(path).read()
    text = strip_comments(raw)
    protos = {}
    # a declaration: return type, name, ( params ) ;  (no bodies in this header)
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b([A-Za-z_]\w*)\s*\(([^;{}()]*)\)\s*;", text):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        ret = " ".join(ret.split()).replace(" *", "*").strip()
        if ret.startswith("typedef") or ret in ("return", ""):
            continue
        line = text.count("\n", 0, m.start(2)) + 1
        plist = []
        p = " ".join(params.split())
        if p and p != "void":
            for item in p.split(","):
                item = item.strip()
                pm = re.match(r"(.*?)([A-Za-z_]\w*)$", item)
                ptype = " ".join(pm.group(1).replace("*", " * ").split()).replace(" *", "*")
                plist.append([ptype, pm.group(2)])
        protos[name] = {"ret": ret, "params": plist, "header_line": line}
    typedefs = {}
    for m in re.finditer(r"typedef\s+struct\s*\{([^}]*)\}\s*(\w+)\s*;", text):
        fields = []
        for decl in m.group(1).split(";"):
            decl = " ".join(decl.split())
            if decl:
                fm = re.match(r"(.*?)\s*\b(\w+)$", decl)
                fields.append([fm.group(1).replace(" *", "*"), fm.group(2)])
        typedefs[m.group(2)] = {"fields": fields, "header_line": text.count("\n", 0, m.start()) + 1}
    for m in re.finditer(r"typedef\s+void\s*\*\s*(\w+)\s*;", text):
        typedefs[m.group(1)] = {"pointer": "void*", "header_line": text.count("\n", 0, m.start()) + 1}
    return protos, typedefs


def scan_go(ref):
    uses = {}
    for pkg in PACKAGES:
        for path in sorted(glob.glob(os.path.join(ref, pkg, "*.go"))):
            if path.endswith("_test.go"):
                continue
            rel = os.path.relpath(path, ref)
            for ln, line in enumerate(open(path), 1):
                code = line.split("//", 1)[0]
                for name in re.findall(r"\bC\.([A-Za-z_]\w*)", code):
                    uses.setdefault(name, []).append(f"{rel}:{ln}")
    return uses


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    protos, typedefs = parse_header(os.path.join(ref, "internal/cgo/metal_bridge.h"))
    uses = scan_go(ref)
    functions, types, unknown = [], {}, []
    for name in sorted(uses):
        if name in NOT_BRIDGE:
            continue
        if name in protos:
            functions.append({"name": name, **protos[name], "go_calls": uses[name]})
        elif name in typedefs:
            types[name] = {**typedefs[name], "go_uses": uses[name][:3]}
        else:
            unknown.append(name)
    if unknown:
        sys.exit(f"C names used by the Go code but not declared in metal_bridge.h: {unknown}")
    out = {
        "source": "internal/cgo/metal_bridge.h prototypes of every C function that "
                  + ", ".join(p + "/*.go" for p in PACKAGES) + " reference (non-test files)",
        "packages": list(PACKAGES),
        "types": types,
        "functions": functions,
    }
    with open(os.path.join(HERE, "cgo_abi.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"{len(functions)} functions, {len(types)} types")


if __name__ == "__main__":
    main()
