"""qvex — MI355X-native kernels for QVex's MTP speculative-decoding verify step.

Python host code mirrors the reference's engine API (engine/kernels.py,
engine/model.py, engine/mtp.py, engine/sampler.py, engine/speculative.py);
every compute op runs in libqvex.so (hand-written HIP for gfx950) through the C
ABI of include/qvex.h. PyTorch only allocates device memory and supplies the
stream.
"""

__version__ = "0.1.0"
