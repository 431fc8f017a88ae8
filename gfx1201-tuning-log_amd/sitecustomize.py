"""Auto-install the hot-path hooks in every Python process that has this directory on its path.

Same chain as vllm-fp8kv/sitecustomize.py:1-24, restricted to the hooks this package provides:
the decode override first, then the linear-op hook, then the prefill hook last so that its
forward wraps the decode override (which wraps vLLM's stock forward).  Each import is guarded:
a process without vLLM, a GPU or the built library is left untouched.
"""
try:
    import fp8kv_override  # noqa: F401
except Exception:
    pass
try:
    import fp8kv_hipw4  # noqa: F401
except Exception:
    pass
try:
    import fp8kv_prefill  # noqa: F401
except Exception:
    pass
