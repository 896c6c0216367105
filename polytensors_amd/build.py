"""Build ``libpolytaylor.so`` (the C-ABI library of the gfx950 kernels) in-tree.

Every ``csrc/*.hip`` file is compiled with ``hipcc --offload-arch=gfx950`` into
an object under ``csrc/_build/``, in parallel, and the objects are linked into
``polytensors_amd/_lib/libpolytaylor.so``. The library links the HIP runtime by
soname (``libamdhip64.so.7``), so inside a process that imported torch first it
binds to the runtime torch already loaded.

Run ``python -m polytensors_amd.build`` (incremental) or ``--force``.
"""

import concurrent.futures
import hashlib
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(CSRC, "_build")
LIB_DIR = os.path.join(HERE, "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libpolytaylor.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed FP32 (v_pk_*_f32) is switched off for all device code.
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC,
    "-Wno-unused-result",
]


def _sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


_INCLUDE_RE = re.compile(rb'^\s*#\s*include\s*"([^"]+)"', re.M)


def _local_includes(path, seen):
    """``path`` and the files its quoted #includes reach, transitively (csrc/ and include/)."""
    if path in seen:
        return
    seen.add(path)
    with open(path, "rb") as fh:
        text = fh.read()
    for name in _INCLUDE_RE.findall(text):
        name = name.decode()
        for base in (os.path.dirname(path), CSRC, INCLUDE):
            candidate = os.path.normpath(os.path.join(base, name))
            if os.path.exists(candidate):
                _local_includes(candidate, seen)
                break


def _object_for(src):
    """Object path tagged with a digest of the source, every local header it reaches, and the flags."""
    files = set()
    _local_includes(src, files)
    h = hashlib.sha256(" ".join(CFLAGS).encode())
    for path in sorted(files):
        with open(path, "rb") as fh:
            h.update(path.encode() + b"\0" + fh.read())
    name = os.path.splitext(os.path.basename(src))[0]
    return os.path.join(OBJ_DIR, f"{name}.{h.hexdigest()[:16]}.o")


def _compile(src, obj):
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj + ".tmp"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature: drop that warning only.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{err}")
    os.replace(obj + ".tmp", obj)
    return err


def build(force=False, jobs=None, verbose=True):
    """Compile the kernels and link the library; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    sources = _sources()
    objects = [_object_for(s) for s in sources]
    todo = [(s, o) for s, o in zip(sources, objects) if force or not os.path.exists(o)]
    jobs = jobs or min(8, os.cpu_count() or 1)
    if todo:
        with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
            futures = {pool.submit(_compile, s, o): s for s, o in todo}
            for fut in concurrent.futures.as_completed(futures):
                warnings = fut.result()
                if verbose:
                    print(f"[polytaylor] compiled {os.path.basename(futures[fut])}", flush=True)
                    if warnings.strip():
                        print(warnings, flush=True)
    stale = [os.path.join(OBJ_DIR, f) for f in os.listdir(OBJ_DIR)
             if f.endswith(".o") and os.path.join(OBJ_DIR, f) not in objects]
    for path in stale:
        os.remove(path)
    if todo or force or not os.path.exists(LIB_PATH):
        tmp = LIB_PATH + ".tmp"
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", tmp]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"link of libpolytaylor.so failed:\n{proc.stderr}")
        os.replace(tmp, LIB_PATH)
        if verbose:
            print(f"[polytaylor] linked {LIB_PATH}", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build(force="--force" in sys.argv)
