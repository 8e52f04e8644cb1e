"""CPU oracle for the bundle-adjustment linearize + Schur path.

THIS PACKAGE IS TEST INFRASTRUCTURE. It is a plain CPU (torch / numpy) restatement of the
reference algorithm (naver/blast3r), written from the reference source text:

  * ``kernels``  -- the five ``cujac`` entry points and ``exp_se3``
                    (src/blast3r/extensions/cujac/sfm_jacobian_rigs.cu,
                     src/blast3r/extensions/cujac/__init__.py)
  * ``solver``   -- ``GaussNewtonSolver`` normal equations, per-leaf damping,
                    Schur reduction, Jacobi-PCG and back-substitution
                    (src/blast3r/inference/ba_solver.py)
  * ``engine``   -- ``lm_step`` / ``bundle_adjustment`` control flow
                    (src/blast3r/inference/engine.py)
  * ``sampling`` -- F sampling: ``bilinear_sampling`` / ``grid_sample`` and
                    ``gather_data_from_dense_tracks`` (src/blast3r/utils/geometry.py,
                    src/blast3r/inference/tracks.py), numpy fp32
  * ``dense``    -- brute-force dense versions (materialised J, dense normal
                    equations, dense Schur) used only to pin the above on tiny
                    problems.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU baseline.
The product path (``blast3r_amd``) never imports, calls or falls back to it.

Parity pinning of each function (what fixes it besides its own formula) is
listed in the module docstrings and exercised by ``tests/test_oracle.py`` and
``tests/test_sampling.py``.
"""
