"""Minimal stand-in for the parts of vLLM's public API that fxpr_vllm's glue
modules import (test infrastructure only; vLLM is not installed here). Class
and function names follow vLLM; behaviour is reduced to what the tests need."""
