"""xfold_cpu_amd: the MI355X (gfx950) HIP backend for xfold's Pairformer and
diffusion-transformer hot operators.

``xfold_cpu_amd.fastnn`` mirrors the reference's ``xfold.fastnn`` operator API and
``xfold_cpu_amd.nn`` its module classes; both run on ``libxfold_hip.so`` (C ABI in
``include/xfold_hip.h``), built by ``python -m xfold_cpu_amd._build``.
"""

__version__ = "0.1.0"
