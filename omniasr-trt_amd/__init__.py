"""omniASR's speculative greedy decoder step on AMD Instinct MI355X (gfx950).

A drop-in for omniasr-trt's decode-step kernels (``omniasr_trt.kernels``) and the decoders built on them:

* ``kernels``  -- the reference's kernel API over hand-written HIP kernels (``libomniasr_mi355x.so``, C ABI in
  ``include/omniasr_mi355x.h``): RoPE + KV append, multi-query split-K verify attention, draft proposal,
  argmax + acceptance / rollback;
* ``decode``   -- ``GreedyDecoder``: static KV cache, HIP-graph steps, continuous-batching host loop;
* ``spec``     -- ``SpecDecoder``: the drafted (speculative) greedy step;
* ``beam``     -- ``BeamDecoder``: batched beam search over shared-context / pointer-indirected caches;
* ``batching`` -- the continuous-batching scheduler, step-graph cache and packed weights the decoders share;
* ``transcribe`` -- ``Transcriber``: segment contexts, the choice of decoder, CTC-frame drafts into the drafted
  decoder (the reference's ``LLMTranscriber`` decoding side);
* ``modeling`` -- the omniASR LLM decoder (fairseq2 parameter names) and its RoPE table;
* ``llm``      -- streaming constants, the repetition stop, CTC-frame drafts.

The directory name is not a Python identifier; the package registers itself (and its modules) under the
importable name ``omniasr_trt_amd`` as well.
"""

import sys as _sys

_ALIAS = "omniasr_trt_amd"
_sys.modules.setdefault(_ALIAS, _sys.modules[__name__])

from . import _lib, kernels, llm, modeling  # noqa: E402
from . import batching, decode, spec  # noqa: E402
from . import beam, transcribe  # noqa: E402

for _name, _mod in (("_lib", _lib), ("kernels", kernels), ("llm", llm), ("modeling", modeling),
                    ("batching", batching), ("decode", decode), ("spec", spec), ("beam", beam),
                    ("transcribe", transcribe)):
    _sys.modules.setdefault(f"{_ALIAS}.{_name}", _mod)

__all__ = ["batching", "beam", "decode", "kernels", "llm", "modeling", "spec", "transcribe"]
