"""No device code of the library writes outside its buffers: the operator
flows of the benchmark harness and of the golden fixtures run in a child
process with the device allocation guards on (PS_DEVICE_GUARD: 4 KiB of a
known pattern before and after every block the library allocates, checked
on the host when the block is freed and at the end), and no guard byte may
change."""
import os
import subprocess
import sys

import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def test_no_device_write_leaves_its_buffer():
    env = dict(os.environ, PS_DEVICE_GUARD="4096")
    r = subprocess.run([sys.executable, os.path.join(HERE, "guard_child.py")], env=env,
                       capture_output=True, text=True, timeout=600)
    say(r.stdout.strip())
    say(r.stderr.strip()[-4000:])
    assert r.returncode == 0, f"child exited with {r.returncode}"
    assert "guard violations: 0" in r.stdout
    assert "ps guard:" not in r.stderr
