"""lit-style tests of the text pipeline (tests/lit/*.mlir), run on the CPU.

Each file's `// RUN:` lines are shell pipelines, as in the reference's
test/Transforms/*.mlir: `frisk-opt` is this package's driver
(`python -m frisk_amd.opt`), `FileCheck` is LLVM's (ROCm ships it), `%s` the
file, `%t` a scratch path and `%S` the file's directory; a stage `not cmd`
expects cmd to fail.  Every RUN line must exit 0 (bash -o pipefail)."""
import os
import re
import shlex
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

LIT = Path(__file__).resolve().parent / "lit"
ROOT = LIT.parents[1]
FILECHECK = shutil.which("FileCheck") or next(
    (p for p in ("/opt/rocm/lib/llvm/bin/FileCheck", "/opt/rocm/llvm/bin/FileCheck")
     if os.path.exists(p)), None)


def run_lines(path: Path):
    lines, cur = [], ""
    for raw in path.read_text().splitlines():
        m = re.match(r"\s*//\s*RUN:\s?(.*)$", raw)
        if not m:
            continue
        part = m.group(1)
        if part.endswith("\\"):
            cur += part[:-1] + " "
            continue
        lines.append(cur + part)
        cur = ""
    return lines


def split_pipeline(cmd: str):
    """Split on `|` outside quotes (not `||`)."""
    stages, buf, quote, i = [], "", None, 0
    while i < len(cmd):
        c = cmd[i]
        if quote:
            buf += c
            if c == quote:
                quote = None
        elif c in "'\"":
            quote = c
            buf += c
        elif c == "|" and cmd[i + 1:i + 2] != "|" and (i == 0 or cmd[i - 1] != "|"):
            stages.append(buf)
            buf = ""
        else:
            buf += c
        i += 1
    stages.append(buf)
    return stages


def expand(cmd: str, path: Path, tmp: Path) -> str:
    opt = f"{shlex.quote(sys.executable)} -m frisk_amd.opt"
    cmd = cmd.replace("%s", shlex.quote(str(path))).replace("%S", shlex.quote(str(path.parent)))
    cmd = cmd.replace("%t", shlex.quote(str(tmp / "t")))
    stages = []
    for st in split_pipeline(cmd):
        st = re.sub(r"(?<![\w-])frisk-opt(?![\w-])", opt, st)
        st = re.sub(r"(?<![\w-])FileCheck(?![\w-])", shlex.quote(FILECHECK), st)
        s = st.strip()
        if s.startswith("not "):
            st = "{ ! " + s[4:] + " ; }"
        stages.append(st)
    return "|".join(stages)


@pytest.mark.skipif(FILECHECK is None, reason="FileCheck is not installed")
@pytest.mark.parametrize("path", sorted(LIT.glob("*.mlir")), ids=lambda p: p.name)
def test_lit(path, tmp_path):
    runs = run_lines(path)
    assert runs, f"{path.name} has no RUN lines"
    env = dict(os.environ, PYTHONPATH=str(ROOT) + os.pathsep + os.environ.get("PYTHONPATH", ""))
    for cmd in runs:
        full = expand(cmd, path, tmp_path)
        r = subprocess.run(["bash", "-o", "pipefail", "-c", full], cwd=tmp_path, env=env,
                           capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, f"RUN: {cmd}\n$ {full}\n{r.stdout[-3000:]}\n{r.stderr[-3000:]}"
