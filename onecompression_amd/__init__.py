"""onecomp-amd: MI355X-native quantized-linear hot path of OneComp.

A drop-in for OneComp's ``mixed_gptq`` and ``dbf`` vLLM plugins (and the
HF-path GPTQ/DBF/MDBF modules): the plugin-facing classes live in
:mod:`onecompression_amd.gptq` and :mod:`onecompression_amd.dbf`; the kernels
are hand-written HIP for gfx950 behind the C ABI of ``include/onecomp_amd.h``.
"""

__version__ = "0.1.0"
