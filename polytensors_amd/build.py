"""Build ``libpolytaylor.so`` (the C-ABI library of the gfx950 kernels) and its
PyTorch registration ``libpolytaylor_torch.so`` in-tree.

Every ``csrc/*.hip`` file is compiled with ``hipcc --offload-arch=gfx950`` into
an object under ``csrc/_build/``, in parallel, and the objects are linked into
``polytensors_amd/_lib/libpolytaylor.so``. The library links the HIP runtime by
soname (``libamdhip64.so.7``), so inside a process that imported torch first it
binds to the runtime torch already loaded. ``csrc/torch_ops.cpp`` (host code:
the ``polytensors_amd::*`` operator schemas and their HIP implementations over
the C ABI) is compiled against the installed torch's headers and linked with
``libpolytaylor.so`` (found beside it) and torch's libraries.

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
TORCH_LIB_PATH = os.path.join(LIB_DIR, "libpolytaylor_torch.so")
TORCH_SRC = os.path.join(CSRC, "torch_ops.cpp")
CXX = os.environ.get("CXX", "g++")
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
    build_torch_ops(force=force or bool(todo), verbose=verbose)
    return LIB_PATH


def _torch_flags():
    import torch
    import torch.utils.cpp_extension as ext

    try:
        incs, libs = ext.include_paths(device_type="cuda"), ext.library_paths(device_type="cuda")
    except TypeError:   # older signature
        incs, libs = ext.include_paths(cuda=True), ext.library_paths(cuda=True)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return ([f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM"] +
            [f"-I{d}" for d in incs], [f"-L{d}" for d in libs] + [f"-Wl,-rpath,{d}" for d in libs])


def build_torch_ops(force=False, verbose=True):
    """Compile csrc/torch_ops.cpp into _lib/libpolytaylor_torch.so (skipped when up to date)."""
    files = set()
    _local_includes(TORCH_SRC, files)
    cflags, ldflags = _torch_flags()
    h = hashlib.sha256(" ".join(cflags + ldflags).encode())
    for path in sorted(files):
        with open(path, "rb") as fh:
            h.update(path.encode() + b"\0" + fh.read())
    stamp = TORCH_LIB_PATH + ".digest"
    digest = h.hexdigest()
    if not force and os.path.exists(TORCH_LIB_PATH) and os.path.exists(stamp):
        with open(stamp) as fh:
            if fh.read().strip() == digest:
                return TORCH_LIB_PATH
    tmp = TORCH_LIB_PATH + ".tmp"
    cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-shared", *cflags, TORCH_SRC, "-o", tmp,
           f"-L{LIB_DIR}", "-lpolytaylor", *ldflags, "-Wl,-rpath,$ORIGIN",
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build of libpolytaylor_torch.so failed:\n{proc.stderr}")
    os.replace(tmp, TORCH_LIB_PATH)
    with open(stamp, "w") as fh:
        fh.write(digest + "\n")
    if verbose:
        print(f"[polytaylor] built {TORCH_LIB_PATH}", flush=True)
    return TORCH_LIB_PATH


if __name__ == "__main__":
    build(force="--force" in sys.argv)
