"""The device-memory pool and its retired list (tensomite.cr_amd/csrc/
tmh_pool.h) under host threads, on the CPU: tests/sanitize/pool_race.cpp
built with g++ and run. Pusher threads give memory back as finalizers do
(RetiredList#push, buffer_pool.cr:98-110: never waiting) while three threads
drain into the pool at once, as tmh_alloc and tmh_sync may on any calling
thread (the C ABI lets any thread call); every pointer must come back exactly
once, and the pool must never hand one out twice. The reference drains from
one thread only (buffer_pool.cr:112-113); drains on several threads must wait
for one another, or a second drain swaps back into use the array the first is
still reading.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_retired_list_and_pool_under_threads(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    exe = tmp_path / "pool_race"
    subprocess.run([gxx, "-O2", "-std=c++17", "-pthread", os.path.join(ROOT, "tests", "sanitize", "pool_race.cpp"),
                    "-o", str(exe)], check=True, capture_output=True)
    for _ in range(3):
        r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stdout + r.stderr
        assert " 0 lost, 0 back more than once, 0 handed out twice" in r.stdout, r.stdout
