"""pip / setuptools entry: build_py also compiles the gfx950 HIP library and the
``flash_hypercons._C`` registration module (``flash-hyperconnections_amd/build.py``)
into the package directory of the build, so wheels and ``pip install`` carry them.

Counterpart of the reference's setup.py:14-24 (a torch CUDAExtension); here the
kernels are plain hipcc objects linked into one shared library that the
registration module loads, as ``__graft_entry__.build()`` does in tree.
"""

import sys
from pathlib import Path

from setuptools import find_packages, setup
from setuptools.command.build_py import build_py

ROOT = Path(__file__).resolve().parent


class BuildWithKernels(build_py):
    def run(self):
        super().run()
        sys.path.insert(0, str(ROOT / "flash-hyperconnections_amd"))
        import build as fh_build  # flash-hyperconnections_amd/build.py

        out_dir = Path(self.build_lib) / "flash_hypercons"
        obj_dir = Path(self.get_finalized_command("build").build_temp) / "flash_hypercons"
        for path in fh_build.build(out_dir=out_dir, obj_dir=obj_dir):
            print(f"built {path}")


setup(
    name="flash-hypercons",
    version="0.1.0",
    description="Small batched matrix exponentials for PyTorch on AMD Instinct MI355X (gfx950)",
    long_description=(ROOT / "README.md").read_text(),
    long_description_content_type="text/markdown",
    python_requires=">=3.10",
    install_requires=["torch"],
    extras_require={"test": ["pytest", "numpy", "scipy"]},
    package_dir={"": "flash-hyperconnections_amd"},
    packages=find_packages("flash-hyperconnections_amd", include=["flash_hypercons", "flash_hypercons.*"]),
    package_data={"flash_hypercons": ["*.so"]},
    cmdclass={"build_py": BuildWithKernels},
)
