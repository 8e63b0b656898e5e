#!/usr/bin/env python3
"""Write the kernel argument table the recording HIP stand-in needs
(hipstub.cpp): for every kernel of the library's real gfx950 build, its
explicit arguments in order, 'g8' for a pointer, 'v<size>' for a by-value
argument.  Read from the code-object metadata of the built objects
(objcopy the .hip_fatbin section, unbundle the gfx950 code object, parse the
amdhsa.kernels notes).

    python kernel_args.py OUT.tsv OBJ.o [OBJ.o ...]
"""
import os
import subprocess
import sys
import tempfile

import yaml

LLVM = "/opt/rocm/llvm/bin"


def kernels_of(obj, tmp):
    fat = os.path.join(tmp, os.path.basename(obj) + ".fatbin")
    co = os.path.join(tmp, os.path.basename(obj) + ".co")
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", obj, fat], check=True)
    subprocess.run([f"{LLVM}/clang-offload-bundler", "--type=o", f"--input={fat}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}", "--unbundle"], check=True)
    notes = subprocess.run([f"{LLVM}/llvm-readelf", "--notes", co], check=True, capture_output=True,
                           text=True).stdout
    start = notes.index("amdhsa.kernels:")
    end = notes.index("amdhsa.target", start)
    lines = notes[notes.rfind("\n", 0, start) + 1:end].splitlines()
    ind = len(lines[0]) - len(lines[0].lstrip())
    doc = yaml.safe_load("\n".join(ln[ind:] for ln in lines))
    for k in doc["amdhsa.kernels"]:
        args = []
        for a in k.get(".args", []):
            kind = a[".value_kind"]
            if kind.startswith("hidden_"):
                continue
            args.append("g8" if kind == "global_buffer" else f"v{a['.size']}")
        yield k[".name"], args


def main():
    out, objs = sys.argv[1], sys.argv[2:]
    rows = {}
    with tempfile.TemporaryDirectory() as tmp:
        for obj in objs:
            for name, args in kernels_of(obj, tmp):
                rows[name] = args
    with open(out, "w") as f:
        for name in sorted(rows):
            f.write(f"{name}\t{','.join(rows[name])}\n")
    print(f"{out}: {len(rows)} kernels")


if __name__ == "__main__":
    main()
