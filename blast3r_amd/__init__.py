"""blast3r_amd: MI355X-native bundle-adjustment linearize + Schur path for BLASt3R.

Drop-in replacements for the reference's BA path:

  * ``blast3r_amd.cujac``      -- the ``blast3r.extensions.cujac`` operator module
  * ``blast3r_amd.ba_solver``  -- ``GaussNewtonSolver`` (fused HIP linearize + Schur + PCG)
  * ``blast3r_amd.engine``     -- ``lm_step`` / ``bundle_adjustment``
  * ``blast3r_amd.data``       -- ``RigsData`` / ``ObservedTracks`` fields used by BA

All compute runs in ``libba_hip.so`` (C ABI, include/ba_hip.h), built in-tree by
``blast3r_amd.build``.
"""
__version__ = '0.1.0'
