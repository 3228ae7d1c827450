"""Build and install ops3d_amd: the gfx950 Flash Deformable 3D Attention library.

`python setup.py build_ext` compiles ops3d_amd/csrc/*.hip with hipcc for gfx950 only (no
hipify, no CUDA headers) into ops3d_amd/libops3d_fda.so; `pip install .` does the same and
installs the `ops3d_amd` package and the `ops3d` alias package.
"""
from setuptools import setup
from setuptools.command.build_ext import build_ext
from setuptools.command.build_py import build_py


class HipBuild(build_ext):
    def run(self):
        from ops3d_amd import _build

        _build.build()


class BuildPyWithLib(build_py):
    def run(self):
        self.run_command("build_ext")
        super().run()


setup(
    name="ops3d_amd",
    version="0.1.0",
    description="MI355X-native Flash Deformable 3D Attention (drop-in for ops3d.flash_deform_attn)",
    packages=["ops3d_amd", "ops3d"],
    package_data={"ops3d_amd": ["libops3d_fda.so", "csrc/*.hip", "csrc/*.h"]},
    cmdclass={"build_ext": HipBuild, "build_py": BuildPyWithLib},
    python_requires=">=3.9",
)
