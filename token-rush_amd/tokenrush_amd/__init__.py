"""tokenrush_amd: the speculative-decoding verify path of token-rush, MI355X-native.

Modules mirror the reference's API for this path:
  quant   - QLinear and the int4 helpers (tokenrush/quant.py)
  gfx950  - the weight-layout backend (the role of tokenrush/marlin.py)
  sample  - SamplingParams / sample (tokenrush/sample.py)
  accept  - the on-device accept/commit of Engine._verify_step (tokenrush/model.py:293-312),
            plus residual rejection sampling and tree accept
All compute runs in the HIP kernels of libtrhip.so (see _lib.py).
"""
