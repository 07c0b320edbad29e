"""Builds ``bux_amd/libbux_amd.so`` from ``bux_amd/csrc`` with hipcc for gfx950.

Run as ``python -m bux_amd.build`` (or through ``__graft_entry__.build()``). Each
source compiles to an object in ``bux_amd/_build/`` in parallel, then one shared
library links them; the library lands next to this file, in-tree, where the loader
(`bux_amd._lib`) finds it.
"""

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIBRARY = os.path.join(HERE, "libbux_amd.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # No packed-float32 instructions: some of their forms have given wrong results on
    # these machines without an error.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def sources() -> list[str]:
    """Return the library's source files."""
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp"))
    )


def _compile(src: str) -> str:
    obj = os.path.join(OUT_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{proc.stdout}\n{proc.stderr}")
    return obj


XLA_SOURCE = os.path.join(HERE, "xla", "xla_ffi.cc")
XLA_LIBRARY = os.path.join(HERE, "libbux_amd_xla.so")


def xla_ffi_include() -> str | None:
    """The XLA FFI headers' include directory: BUX_XLA_FFI_INCLUDE, else jax's own
    (jax.ffi.include_dir()); None where neither is there."""
    env = os.environ.get("BUX_XLA_FFI_INCLUDE")
    if env:
        return env
    try:
        import jax.ffi  # noqa: PLC0415 (optional: jax is absent where bux_amd is used alone)
        return jax.ffi.include_dir()
    except Exception:  # noqa: BLE001 (no jax, or one without the FFI)
        return None


def build_xla(verbose: bool = True) -> str | None:
    """Build the XLA FFI handlers (libbux_amd_xla.so, linked to libbux_amd.so) where the
    XLA FFI headers are; return its path, or None where they are not."""
    inc = xla_ffi_include()
    if inc is None or not os.path.exists(os.path.join(inc, "xla", "ffi", "api", "ffi.h")):
        if verbose:
            print("XLA FFI headers not found: libbux_amd_xla.so not built "
                  "(set BUX_XLA_FFI_INCLUDE or install jax)", file=sys.stderr)
        return None
    cmd = [HIPCC, "-std=c++17", "-O2", "-fPIC", "-shared", "-I", os.path.join(ROOT, "include"),
           "-I", inc, XLA_SOURCE, "-L", HERE, "-lbux_amd", "-Wl,-rpath,$ORIGIN", "-o", XLA_LIBRARY]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"the XLA FFI handlers failed to build:\n{proc.stdout}\n{proc.stderr}")
    return XLA_LIBRARY


def build(verbose: bool = True) -> str:
    """Compile every source and link the shared library (and, where the XLA FFI headers
    are, the handlers' library); return the library's path."""
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIBRARY + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(srcs)} sources", file=sys.stderr)
    build_xla(verbose)
    return LIBRARY


if __name__ == "__main__":
    build()
