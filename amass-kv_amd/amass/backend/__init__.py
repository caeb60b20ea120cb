"""vLLM-ROCm plugin boundary (reference: src/amass/backend/).

  register.py   register(): patches RocmPlatform.get_attn_backend_cls so the chosen
                decoder backend is subclassed with the AMASS impl and builder
  attn.py       impl mixin: pure single-token decode -> Stage A select + Stage B decode
  builder.py    metadata-builder mixin: lazy state, summary refresh gate, derive
  _runtime.py   the AmassConfig singleton, state construction, select / decode dispatch

Nothing here imports vLLM at module import time; register() does.
"""
