"""Hardware-ceiling probes (empty launch, one-pass HBM read, fp16 MFMA rate)
that the kernels' measured rates are compared against; see run.py."""
