"""Import path of the sc_amd package for the code_gen command-line tools."""
import os
import sys

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CODE_GEN = os.path.join(PKG_ROOT, "code_gen")
for _p in (PKG_ROOT, CODE_GEN):
    if _p not in sys.path:
        sys.path.insert(0, _p)
