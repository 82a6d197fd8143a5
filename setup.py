"""Build entry point mirroring the reference's ``python setup.py build_ext --inplace``
(reference setup.py:46-153): hipcc compiles the gfx950 kernels and the C ABI into
``libmuon_polar.so``; the torch operator ``_C.so`` links it.  Both land in place, next to
``muon_fusion_ascend950_amd/__init__.py``."""

from setuptools import Command, setup
from setuptools.command.build_ext import build_ext


class InPlaceHipBuild(build_ext):
    def run(self):
        # Load the build script by path: importing the package would load the native
        # library that is being built (missing or stale at this point).
        import importlib.util
        from pathlib import Path

        path = Path(__file__).resolve().parent / "muon_fusion_ascend950_amd" / "_build.py"
        spec = importlib.util.spec_from_file_location("muon_fusion_ascend950_amd_build", path)
        module = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(module)
        module.build(verbose=True)


setup(
    name="muon_fusion_ascend950_amd",
    version="0.1.1",
    packages=["muon_fusion_ascend950_amd", "muon_ascend950"],
    package_data={"muon_fusion_ascend950_amd": ["_C.so", "libmuon_polar.so"]},
    cmdclass={"build_ext": InPlaceHipBuild},
)
