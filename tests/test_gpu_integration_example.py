"""The Python example of INTEGRATION.md section 3 runs as written (the
scan plan and the DeviceApi consumer kernel), and its results are right."""
from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

DOC = Path(__file__).resolve().parent.parent / "INTEGRATION.md"


def test_python_example_runs(capsys):
    text = DOC.read_text()
    section = text[text.index("## 3. Python"):text.index("## 4. C / C++")]
    code = re.search(r"```python\n(.*?)```", section, re.S).group(1)
    env: dict = {}
    exec(compile(code, "INTEGRATION.md", "exec"), env)
    dev, x, out = env["dev"], env["x"], env["out"]
    dev.synchronize()
    n = 1 << 20
    got = dev.download_owned(out)
    assert np.array_equal(got, np.arange(n, dtype=np.uint32) + np.uint32(7))
    printed = capsys.readouterr().out
    assert printed.strip() == str(np.array([0, 0, 1, 3], dtype=np.uint32))
