"""Host side of the MI355X fused Q4 decode step (Python mirror of engine/infer.js).

    pgw     PGW1 container reader/writer, quantisers, synthetic models
    abi     ctypes binding of libmllm (include/mllm.h)
    engine  PetitGPT API over libmllm (forwardPrompt / forwardDecode / generate)
    tokenizer  byte-level BPE + chat templates (engine/tokenizer.js); import
               mllm.tokenizer where text is needed
"""
from . import abi, pgw  # noqa: F401
from .engine import PetitGPT, argmax, argmax_gpt2, lookup_draft  # noqa: F401
