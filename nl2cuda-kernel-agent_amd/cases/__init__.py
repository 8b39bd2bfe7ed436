"""Algorithm cases.  Each sub-package exposes ``CASE`` (framework.case.Case)
and an ``op`` module with ``candidate(inputs, params)`` backed by HIP."""
