"""tinygpt_amd -- MI355X-native decode-time logits processing and sampling.

The product is libtgs_sampler.so (C ABI in include/tgs_sampler.h): gfx950
HIP kernels for penalties, temperature, the grammar mask, top-k, top-p, the
categorical draw and speculative verification.  This package holds the
kernels' sources (csrc/), the in-tree build, a ctypes binding (`Sampler`,
`sample_noalloc`), the host grammar compilers whose automata fill
mask-table rows on the device (`grammar` for GBNF, `json_schema` for JSON
schemas), and the synthetic workloads of the benchmark configurations
(`workloads`).
"""
from ._lib import (  # noqa: F401
    EXPORTS,
    ROW_PARAMS_DTYPE,
    TGS_BF16,
    TGS_EALLMASKED,
    TGS_EINVAL,
    TGS_F32,
    TGS_FLAG_GREEDY,
    TGS_OK,
    TgsError,
    load,
)
from .sampler import Sampler, batch_hint, make_params, params_to_device, sample_noalloc  # noqa: F401
