"""`attn_kernel` drop-in package (a namespace directory in the reference).  The package path is
extended over every other `attn_kernel` directory on sys.path, so the drop-in modules here win
and any other kernel module named by a benchmark's `--kernel` string still resolves to the
reference's copy beside the script."""
from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)
