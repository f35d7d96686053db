"""The CPU restatement under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

oracle/sanitize_check.c drives every entry point of oracle/fh_oracle.c over
n = 1..32, both directions, both combine contractions and inputs with zeros,
subnormals, values near FP32's maximum, infinities and NaNs; this builds it
together with the oracle with gcc's sanitizers (any report aborts the run) and
requires a clean run.  The batched forward and the parameters entry point must
also agree on every squaring count.
"""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SAN = ["-fsanitize=address,undefined,float-cast-overflow", "-fno-sanitize-recover=all"]


def _gcc():
    return shutil.which("gcc")


def test_oracle_runs_clean_under_sanitizers(tmp_path):
    gcc = _gcc()
    if gcc is None:
        pytest.skip("gcc not available")
    probe = tmp_path / "probe.c"
    probe.write_text("int main(void) { return 0; }\n")
    if subprocess.run([gcc, *SAN, str(probe), "-o", str(tmp_path / "probe")], capture_output=True).returncode:
        pytest.skip("gcc has no sanitizer runtime here")
    exe = tmp_path / "sanitize_check"
    build = subprocess.run(
        [gcc, "-O1", "-g", "-std=c11", "-ffp-contract=off", *SAN, str(ROOT / "oracle" / "fh_oracle.c"),
         str(ROOT / "oracle" / "sanitize_check.c"), "-lm", "-o", str(exe)],
        capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-2000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300,
                         env={"ASAN_OPTIONS": "detect_leaks=1", "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert run.returncode == 0, (run.stdout + run.stderr)[-3000:]
    assert "0 failures" in run.stdout
