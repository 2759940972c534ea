"""Host-side policies of the runtime, exercised with g++ (no GPU).

The device pool's caching policy (acfun_amd/csrc/pool.hpp), exercised on
the host with a mock backend: one stream reuses its blocks with no
synchronization, a caller creating and dropping a stream per call grows the
pool only up to the reclaim threshold, a block of another stream is handed out
only after a device sync, and the out-of-memory path releases the cache after
a device sync."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def test_pool_policy(tmp_path):
    exe = tmp_path / "pool_check"
    src = os.path.join(HERE, "pool", "pool_check.cpp")
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-fsanitize=address,undefined",
                        "-o", str(exe), src], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.fail("pool_check did not build:\n" + r.stderr)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.strip() == "ok"


def test_tune_adoption_rule(tmp_path):
    """The tile search adopts a candidate only when it beats the built-in
    choice by more than 3% (acfun_amd/csrc/tune_rule.hpp), as the reference
    vetoes tuned blockings that regress more than 3% (src/autotune.cpp:147,212)."""
    exe = tmp_path / "tune_rule_check"
    src = os.path.join(HERE, "tune_rule", "tune_rule_check.cpp")
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-o", str(exe), src],
                       capture_output=True, text=True)
    if r.returncode != 0:
        pytest.fail("tune_rule_check did not build:\n" + r.stderr)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.strip() == "ok"
