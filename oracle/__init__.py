"""CPU oracle for the chunked causal LTX attention path -- TEST INFRASTRUCTURE ONLY.

This package restates, op for op on the CPU (PyTorch float32/float64 and numpy),
the reference TaoMate functions the MI355X kernels replace.  Every function
cites the reference ``file:line`` it follows.  It is imported only by
``tests/``, by ``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of
``bench.py`` -- always as the checker or the timed CPU baseline, never as the
thing measured or shipped.  The product package (``taomate_amd``) never imports
it and fails loudly when its HIP library is missing.

How each part is pinned (beyond re-typing the reference):

* ``rope``: the float32 table equals a float64 closed form of the same
  positions/frequencies to <= 2e-6 abs; special cases (pad entries are
  cos 1 / sin 0, frame 0 time = 0.5/24 s, ``ind[0] = pi/2``, spatial midpoints)
  are asserted directly; rotation preserves pair norms; ``sin = 0`` is the
  identity.
* ``attention``: full-row RMSNorm against a float64 textbook formula; SDPA
  against a brute-force float64 softmax on tiny and real shapes; key
  permutation invariance; additive ``-inf`` mask equals key removal; a
  planted transposed-operand mistake is shown to fail the check.
* ``cache``: the reference's own docstring known answers for
  ``compute_av_blocks`` / ``compute_aligned_audio_frames``
  (ltx_causal/attention/mask_builder.py:129-134, :252-255); eviction plans
  checked against brute force over token-id tensors.
* ``fp8``: all 256 e4m3fn codes round-trip; rounding of midpoints is to even;
  saturation at 448.
* ``dit``: sinusoid and tanh-GELU closed forms; one-hot modulation tables land
  every value in its slot; with zeroed attention outputs, and with one video
  and one audio token, the dual-stream block has closed forms that fix the
  order of its residuals.
* ``runtime``: the 3-step denoise with zeroed output heads is a closed form in
  the noise tape and the sigmas; renorm, colour correction, commit, memory
  update and retention are checked in their order, each check also run on a
  mutant carrying a plausible slip; the refresh's block selection and global
  positions are known answers over five layouts.
* ``memory``, ``stream``: pooling, resampling, gate and EMA + tether steps from
  their definitions and special cases; the stream replay is composed only of
  the functions above.

The reference's Python itself was not imported: every function above is pinned
by these checks, so no golden vectors had to be generated from it.
"""
