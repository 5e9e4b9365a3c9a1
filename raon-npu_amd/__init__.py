"""raon-npu_amd: the quantized-MoE hot path of raon-npu on MI355X (gfx950).

Layout of the package:

* ``csrc/``       -- HIP kernels and the C ABI (built into ``librmoe.so``)
* ``build.py``    -- hipcc build of ``librmoe.so`` in this directory
* ``_lib.py``     -- ctypes binding of the C ABI (include/raon_moe.h)
* ``device.py``   -- context / matrix / MoE-layer objects over the ABI
* ``backend.py``  -- ``GpuBackend``: the reference Backend interface for the MoE path
* ``geometry.py`` -- bundle geometry (kernels/moe/pack.py, parameterised)

The directory name contains a hyphen, so entry points load it under the import
name ``raon_npu_amd`` (see ``load_package`` in ``__graft_entry__.py``).
"""

from .geometry import BASELINE, RAON_1_MINI, MoeGeometry  # noqa: F401

__all__ = ["BASELINE", "RAON_1_MINI", "MoeGeometry", "GpuBackend", "Context"]


def __getattr__(name):
    # Defer loading the HIP library until a device object is asked for.
    if name == "GpuBackend":
        from .backend import GpuBackend

        return GpuBackend
    if name == "Context":
        from .device import Context

        return Context
    raise AttributeError(name)
