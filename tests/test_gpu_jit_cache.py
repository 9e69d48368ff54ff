"""The on-disk code-object cache of fused chains (CLOVE_JIT_CACHE).

Each case runs fresh processes (the in-memory cache would hide the disk):
the first compiles the chain with hipRTC and writes its code object, a
later one loads it and compiles nothing, and both give the same bits.  A
damaged file (its header, or code bytes that fail the checksum), one that
others may write, and one reached through a symbolic link are ignored and
replaced; CLOVE_JIT_CACHE=0 writes nothing.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHILD = (
    "import sys; sys.path.insert(0, %r)\n"
    "import numpy as np, clove_amd as ca\n"
    "ca.init(0)\n"
    "x = ca.tensor(np.arange(8192, dtype=np.float32) / 4096 - 1)\n"
    "y = ca.tensor(np.linspace(-3, 3, 8192, dtype=np.float32))\n"
    "(out,) = ca.fused_chain([('mul', -1, -2), ('gelu', 0), ('add', 1, -1)], [x, y])\n"
    "h = out.numpy()\n"
    "c, d = ca.jit_stats()\n"
    "print(c, d, h.tobytes().hex(), flush=True)\n" % ROOT)


def run(env):
    r = subprocess.run([sys.executable, "-c", CHILD], capture_output=True, text=True, timeout=180,
                       env=env)
    assert r.returncode == 0, (r.returncode, r.stdout[-500:], r.stderr[-2000:])
    compiled, loaded, data = r.stdout.split()
    return int(compiled), int(loaded), data


def test_chain_code_object_reused_across_processes(tmp_path):
    cache = tmp_path / "jit"
    env = dict(os.environ, CLOVE_JIT_CACHE=str(cache))
    compiled, loaded, first = run(env)
    assert (compiled, loaded) == (1, 0)
    files = sorted(cache.glob("*.co"))
    assert len(files) == 1 and not list(cache.glob("*.tmp*"))
    compiled, loaded, again = run(env)
    assert (compiled, loaded) == (0, 1) and again == first
    assert (files[0].stat().st_mode & 0o777) == 0o600
    assert (cache.stat().st_mode & 0o777) == 0o700
    # a damaged object is ignored: compiled again, rewritten, then reused
    files[0].write_bytes(b"CLVJIT02 not a code object")
    compiled, loaded, again = run(env)
    assert (compiled, loaded) == (1, 0) and again == first
    compiled, loaded, again = run(env)
    assert (compiled, loaded) == (0, 1) and again == first
    # the key matches but the code bytes are damaged: the checksum rejects
    # them, so the chain is compiled again and the file rewritten
    good = files[0].read_bytes()
    data = bytearray(good)
    klen = int.from_bytes(data[8:16], "little")
    code_at = 16 + klen + 16  # magic, key length, key, code length, checksum
    data[code_at + 100] ^= 0x40
    files[0].write_bytes(bytes(data))
    compiled, loaded, again = run(env)
    assert (compiled, loaded) == (1, 0) and again == first
    compiled, loaded, again = run(env)
    assert (compiled, loaded) == (0, 1) and again == first
    # a file others may write is never read (it may have been planted) ...
    files[0].chmod(0o620)
    compiled, loaded, again = run(env)
    assert (compiled, loaded) == (1, 0) and again == first
    assert (files[0].stat().st_mode & 0o777) == 0o600  # replaced by a private one
    # ... nor one reached through a symbolic link
    elsewhere = tmp_path / "planted.co"
    elsewhere.write_bytes(good)
    files[0].unlink()
    files[0].symlink_to(elsewhere)
    compiled, loaded, again = run(env)
    assert (compiled, loaded) == (1, 0) and again == first
    assert not files[0].is_symlink() and elsewhere.read_bytes() == good


def test_cache_off_writes_nothing(tmp_path):
    home = tmp_path / "home"
    home.mkdir()
    env = dict(os.environ, CLOVE_JIT_CACHE="0", HOME=str(home))
    env.pop("XDG_CACHE_HOME", None)
    for _ in range(2):
        compiled, loaded, _ = run(env)
        assert (compiled, loaded) == (1, 0)
    # (the ROCm toolchain may keep caches of its own under HOME)
    assert not list(home.rglob("clove_hip")) and not list(home.rglob("*.co"))
