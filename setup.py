"""Build entry point (drop-in for the reference's setup.py).

`python setup.py build_ext --inplace` compiles libwush_int4.so (HIP, gfx950)
and the torch module wush_int4_kernel_amd._C in place; `my_int4` then imports
them.  The compile steps live in wush_int4_kernel_amd/_build.py.
"""
import os

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
        # load the build script by path: importing the package would import
        # its (not yet built) native module
        import importlib.util
        spec = importlib.util.spec_from_file_location(
            "wush_int4_kernel_amd_build", os.path.join(HERE, "wush_int4_kernel_amd", "_build.py"))
        build = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(build)
        for path in build.build(verbose=True):
            print("built", path)


setup(
    name="my_int4",
    version="0.1.0",
    description="WUSH INT4 W4A4 inference path for MI355X (gfx950)",
    packages=["my_int4", "wush_int4_kernel_amd"],
    cmdclass={"build_ext": BuildExtInPlace},
)
