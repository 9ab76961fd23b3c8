"""pagedbatch_amd: an MI355X (gfx950) token sampler for pagedbatch's sampling step.

Drop-in for ``pagedbatch.sampling.sample_token`` (pagedbatch/sampling.py:10-27) plus a
batched ``sample`` that takes all rows of one engine step at once. The arithmetic runs in
hand-written HIP kernels (``csrc/pbsample.hip``) behind the C ABI declared in
``include/pbsample.h``; this package is the Python host side: parameter packing, the
per-row uniforms drawn from the caller's seeded generators, and the ctypes binding.
"""

from .config import SamplingParams
from .sampling import SamplerError, SamplingGraph, sample, sample_and_finish, sample_token

__version__ = "0.2.0"

__all__ = ["SamplingParams", "SamplerError", "SamplingGraph", "sample", "sample_and_finish", "sample_token"]
