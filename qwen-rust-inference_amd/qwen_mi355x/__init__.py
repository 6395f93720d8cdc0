"""Host side of the MI355X decode/prefill bridge for the Qwen3.5 hybrid:
model configs and tensor sets (model.py) and the bindings of the host engine
and the gfx950 bridge (engine.py)."""
from . import model  # noqa: F401
