"""MI355X transducer greedy-decode hot path for parakeet.cpp decoders.

The product is the C-ABI library built from ``csrc/`` (``libparakeet_hip.so``)
and the C++ decoder API above it.  This Python package holds the ctypes
binding (``pk``), the GGUF container code (``gguf``) and the seeded synthetic
checkpoint generator (``synth``) used by the tests and the benchmark.
"""
