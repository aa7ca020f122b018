"""`import cmpext3` drop-in: the reference's module name, served by cmp_ext_amd."""
from cmp_ext_amd import *  # noqa: F401,F403
from cmp_ext_amd import extension_path, version  # noqa: F401
