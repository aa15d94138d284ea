"""CPU checks of the decode replay switch (prana_decode_replay_enabled).

Replays of the captured decode step are refused whenever a profiling tool is
loaded into the process, since under rocprofv3's kernel tracing a replaying
process crashed in host code inside hipGraphLaunch. Each case runs in a fresh
process (the decision is made once per process); no GPU work is issued."""
import os
import subprocess
import sys
import textwrap

import pytest

from prana_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROBE = textwrap.dedent("""
    import ctypes, sys
    for path in sys.argv[1:]:
        ctypes.CDLL(path)          # a library mapped before the first query
    lib = ctypes.CDLL({lib!r})
    print(lib.prana_decode_replay_enabled())
""").format(lib=_lib.LIB_PATH)


def replay_enabled(env_extra=None, preload=()):
    env = {k: v for k, v in os.environ.items()
           if not k.startswith("ROCPROF_") and k not in ("ROCP_TOOL_LIBRARIES", "HSA_TOOLS_LIB",
                                                          "PRANA_DECODE_GRAPH")}
    env.update(env_extra or {})
    r = subprocess.run([sys.executable, "-c", PROBE, *preload], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    return int(r.stdout.strip().splitlines()[-1])


@pytest.fixture(scope="module")
def fake_tool(tmp_path_factory):
    """An empty shared library whose file name is the rocprofv3 tool's."""
    d = tmp_path_factory.mktemp("tool")
    src, so = d / "empty.c", d / "librocprofiler-sdk-tool.so.1"
    src.write_text("int prana_test_empty_tool_symbol(void) { return 0; }\n")
    subprocess.run(["gcc", "-shared", "-fPIC", "-o", str(so), str(src)], check=True)
    return str(so)


@pytest.fixture(scope="module")
def fake_register(tmp_path_factory):
    """The registration library every HIP process maps does not count."""
    d = tmp_path_factory.mktemp("reg")
    src, so = d / "empty.c", d / "librocprofiler-register.so.0"
    src.write_text("int prana_test_empty_register_symbol(void) { return 0; }\n")
    subprocess.run(["gcc", "-shared", "-fPIC", "-o", str(so), str(src)], check=True)
    return str(so)


def test_replay_on_by_default(fake_register):
    assert replay_enabled() == 1
    assert replay_enabled(preload=[fake_register]) == 1


@pytest.mark.parametrize("var", ["ROCPROF_KERNEL_TRACE", "ROCPROF_OUTPUT_PATH"])
def test_replay_off_with_profiler_settings(var):
    # (ROCP_TOOL_LIBRARIES / HSA_TOOLS_LIB name libraries the runtime loads at
    # start-up, so they are not set to dummies here)
    assert replay_enabled({var: "1"}) == 0


def test_replay_off_with_profiler_library_mapped(fake_tool):
    assert replay_enabled(preload=[fake_tool]) == 0


def test_replay_off_by_switch():
    assert replay_enabled({"PRANA_DECODE_GRAPH": "0"}) == 0
    assert replay_enabled({"PRANA_DECODE_GRAPH": "1"}) == 1
