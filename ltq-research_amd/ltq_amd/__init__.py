"""MI355X-native (gfx950) implementation of the LTQ TCQ Viterbi quantizer path: HIP kernels behind a C ABI
(include/ltq_hip.h) and a Python surface that mirrors the reference's (src/tcq_proto.py, src/liqk_v2.py,
src/ltq_format.py, src/ltq_file.py)."""
