"""Load the package binding against the test-only host-emulation library
(tests/emu/libq35emu.so) instead of libq35hip.so. Used only when the test
session sets Q35_EMULATION_LIB; the product binding itself never loads it."""
import importlib.util
import os
import sys
import types

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))


def load_twin(lib_path):
    src_path = os.path.join(ROOT, "qwen35-cpu_amd", "__init__.py")
    src = open(src_path).read()
    marker = 'LIB_PATH = os.path.join(HERE, "libq35hip.so")'
    assert marker in src
    src = src.replace(marker, f"LIB_PATH = {os.path.abspath(lib_path)!r}")
    mod = types.ModuleType("qwen35_cpu_amd_emulated")
    mod.__file__ = src_path
    sys.modules[mod.__name__] = mod
    exec(compile(src, src_path, "exec"), mod.__dict__)
    return mod
