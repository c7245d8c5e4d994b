"""CPU-only: the arena side table and the node registry (pico_amd/host/arena.c)
under AddressSanitizer.

Tensors and arenas allocated the way pico allocates them -- a calloc'd 64-byte
PicoTensor (src/tensor.c:44-84), tensors packed back to back in an arena block,
a malloc'd 16-byte two-pointer Arena (src/arena.h:38-64) -- pass through the
node lookup and arena_alloc_device / arena_device_reset / arena_device_release.
A read or write one byte outside them fails the run.  The host test links
arena.c alone, with host stand-ins for the device allocator, so no GPU is
involved.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _build(tmp_path, extra):
    exe = str(tmp_path / "registry_host_test")
    cmd = ["gcc", "-std=c11", "-g", "-O1", "-Wall", "-Wextra", "-Wno-unused-parameter",
           "-pthread", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(ROOT, "pico_amd", "host"),
           os.path.join(ROOT, "pico_amd", "host", "arena.c"),
           os.path.join(ROOT, "tests", "host", "registry_host_test.c"), "-o", exe, *extra]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_registry_and_foreign_arena_under_asan(tmp_path):
    exe = _build(tmp_path, ["-fsanitize=address", "-fno-omit-frame-pointer"])
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "registry host test ok" in r.stdout
    assert "AddressSanitizer" not in r.stderr


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_arena_context_and_registry_threads_under_tsan(tmp_path):
    """Eight threads with their own arena context stacks (pico's
    tests/test_arena.c:160-247) registering and dropping nodes in the shared
    registry at once: ThreadSanitizer reports no race."""
    exe = _build(tmp_path, ["-fsanitize=thread"])
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "registry host test ok" in r.stdout
    assert "ThreadSanitizer" not in r.stderr


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_sanitizer_catches_a_read_past_a_pico_tensor(tmp_path):
    """The check above is only as good as the sanitizer: reading the byte after
    a calloc'd 64-byte tensor, as a magic-number test at offset 64 would, is
    reported here."""
    src = tmp_path / "probe.c"
    src.write_text(
        "#include <stdint.h>\n#include <stdlib.h>\n"
        "int main(void) { unsigned char* t = calloc(1, 64);\n"
        "  volatile uint32_t magic = *(uint32_t*)(t + 64); (void)magic; free(t); return 0; }\n")
    exe = str(tmp_path / "probe")
    subprocess.run(["gcc", "-g", "-fsanitize=address", str(src), "-o", exe], check=True,
                   capture_output=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode != 0
    assert "heap-buffer-overflow" in r.stderr
