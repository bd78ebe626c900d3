"""Build entry point (drop-in for the reference's setup.py).

`python setup.py build_ext --inplace` compiles libwush_int4.so (HIP, gfx950)
and the torch module wush_int4_kernel_amd._C in place; `my_int4` then imports
them.  The compile steps live in wush_int4_kernel_amd/_build.py.
"""
import os
import sys

from setuptools import Command, setup

HERE = os.path.dirname(os.path.abspath(__file__))


class BuildExtInPlace(Command):
    description = "compile the HIP library and the torch module in place"
    user_options = [("inplace", "i", "accepted for compatibility; builds are always in place")]

    def initialize_options(self):
        self.inplace = True

    def finalize_options(self):
        pass

    def run(self):
        sys.path.insert(0, HERE)
        from wush_int4_kernel_amd import _build
        for path in _build.build(verbose=True):
            print("built", path)


setup(
    name="my_int4",
    version="0.1.0",
    description="WUSH INT4 W4A4 inference path for MI355X (gfx950)",
    packages=["my_int4", "wush_int4_kernel_amd"],
    cmdclass={"build_ext": BuildExtInPlace},
)
