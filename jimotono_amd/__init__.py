"""jimotono_amd -- the quantised MoE matmul path of JIMOTONO on AMD MI355X.

The product is the C-ABI shared library ``libjimotono_hip.so`` built from
``csrc/`` (gfx950 HIP kernels + C11 host layer); its prototypes are in
``include/jimotono/*.h``. This package only locates and loads it and offers
thin ctypes wrappers (``jimotono_amd.api``) with the reference's names for
tests and benchmarks. There is no CPU fallback: importing ``api`` without
the built library raises.
"""
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libjimotono_hip.so")

__all__ = ["HERE", "LIB_PATH"]
