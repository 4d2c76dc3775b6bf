import os

# Where the built library lives: tokengate_amd/build.py writes it there and keybias.py loads it
# from there.  FA2BIAS_SITE overrides both at once (kernels/fa2bias/site_path.py:5).  The default
# is inside the package so the built library travels with the source tree.
_DEFAULT_SITE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_site")
SITE = os.path.expanduser(os.environ.get("FA2BIAS_SITE", _DEFAULT_SITE))
BUILD_INFO = "BUILD_INFO.json"
# Bumped when the library gains an entry point callers rely on. 2: key bias on the varlen
# entry points (kernels/fa2bias/site_path.py:7-8).
ABI = 2
LIB_NAME = "libtokengate_hip.so"
