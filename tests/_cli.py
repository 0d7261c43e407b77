"""Running the reference's own CLI and bench -- TEST INFRASTRUCTURE.

oracle/_ref/quillm is the unmodified reference CLI; oracle/_ref/quillm-hip and quillm-bench-hip are
the reference's CLI and bench built with oracle/hip_integration.patch (the "hip" ISA of
INTEGRATION.md), linked against quillm_amd/libqmhip.so (oracle/Makefile, target refhip)."""
import os
import subprocess

from _bind import REF_DIR

QUILLM = os.path.join(REF_DIR, "quillm")
QUILLM_HIP = os.path.join(REF_DIR, "quillm-hip")
BENCH_HIP = os.path.join(REF_DIR, "quillm-bench-hip")
PROMPT = "Once upon a time, there was a little"


def run_cli(exe, model, *args, env=None, timeout=300):
    """(exit code, stdout bytes, stderr text) of `exe run model args...`."""
    e = dict(os.environ)
    e.pop("QUILLM_ISA", None)
    if env:
        e.update(env)
    r = subprocess.run([exe, "run", model, *args], capture_output=True, env=e, timeout=timeout)
    return r.returncode, r.stdout, r.stderr.decode(errors="replace")
