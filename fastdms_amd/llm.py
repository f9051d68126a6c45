"""Public entry point (mirror of fastdms/llm.py): ``LLM(model, **config).generate(...)``."""
from .engine.llm_engine import LLMEngine


class LLM(LLMEngine):
    pass
