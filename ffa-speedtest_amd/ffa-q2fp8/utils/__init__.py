"""`utils` of ffa-q2fp8 (a namespace directory in the reference: ffa-q2fp8/utils has no
__init__.py).  This directory ships only `load.py`; the benchmark scripts also import
`utils.bench`, `utils.cache`, `utils.flash` and `utils.plot` (run_attn_bench_q2.py:12-16,
run_attn_bench_q2_cudagraph.py:13-15).  A regular package would hide the reference's directory,
so the package path is extended over every other `utils` directory on sys.path: `utils.load`
resolves here (first entry), every other module to the reference's copy beside the script."""
from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)
