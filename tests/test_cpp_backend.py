"""The C++ Backend-shaped adapter (include/ggq_backend.h), compiled with g++
against libggq_hip.so and the oracle, driven the way ggnpu's caller drives a
Backend."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "tests", "cpp", "_build")
EXE = os.path.join(BUILD, "backend_test")


@pytest.fixture(scope="module")
def exe():
    from oracle import oracle
    oracle.lib()  # builds liboracle.so if needed
    os.makedirs(BUILD, exist_ok=True)
    lib_dir = os.path.join(ROOT, "ggnpu_amd", "lib")
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "oracle"),
                    os.path.join(ROOT, "tests", "cpp", "backend_test.cpp"), "-o", EXE,
                    "-L", lib_dir, "-lggq_hip", os.path.join(ROOT, "oracle", "liboracle.so"),
                    f"-Wl,-rpath,{lib_dir}", f"-Wl,-rpath,{os.path.join(ROOT, 'oracle')}"], check=True)
    return EXE


def test_backend_adapter_without_device(exe):
    r = subprocess.run([exe, "cpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.gpu
def test_backend_adapter_parity(exe):
    r = subprocess.run([exe, "gpu"], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
