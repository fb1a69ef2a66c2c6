"""The tests' .cellm writer: the package's own (cellm_amd.cellm_file.write_cellm,
llama_header), importable without the GPU."""
from cellm_amd.cellm_file import llama_header, write_cellm  # noqa: F401
