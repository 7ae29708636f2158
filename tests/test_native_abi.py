"""The C ABI without a GPU: the in-tree library loads, exports every entry point the header
declares, and the Python binding's signatures and struct mirror the header. No compute call is
made (those need the GPU and live in the ``gpu``-marked tests)."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

from sglang_omni_amd import _native as N

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "omni_codec.h"


def _header_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(omni_\w+)\s*\(", text, flags=re.M))


def _header_struct_fields(name: str) -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, flags=re.S).group(1)
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        names = decl.split(None, 1)[1] if not decl.startswith("const") else decl.split(None, 2)[2]
        for part in names.split(","):
            fields.append(part.strip().lstrip("*").strip())
    return fields


def test_library_is_built_in_tree():
    assert N.LIB_PATH.exists(), "run __graft_entry__.build() first"
    assert N.LIB_PATH.parent.name == "sglang_omni_amd"


def test_library_exports_every_declared_entry_point():
    declared = _header_functions()
    assert {"omni_rvq_gather_sum", "omni_conv1d_fused", "omni_single_output_conv",
            "omni_history_exchange", "omni_overlap_exchange"} <= declared
    out = subprocess.run(["nm", "-D", "--defined-only", str(N.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (omni_\w+)", out))
    assert declared <= exported, f"not exported: {sorted(declared - exported)}"


def test_binding_covers_the_header_and_loads():
    assert set(N.SIGNATURES) == _header_functions()
    lib = N.load_library()
    for name in N.SIGNATURES:
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)
    assert lib.omni_codec_abi_version() == N.ABI_VERSION == 11
    assert lib.omni_codec_error_string(N.OK) == b"ok"
    assert b"invalid" in lib.omni_codec_error_string(1)


def test_conv_args_struct_mirrors_the_header():
    assert [f[0] for f in N.ConvArgs._fields_] == _header_struct_fields("omni_conv_args")


def test_dtype_and_activation_codes_match_the_header():
    text = HEADER.read_text()

    def value(name: str) -> int:
        return int(re.search(rf"\b{name}\s*=\s*(\d+)", text).group(1))

    assert N.DTYPE_F32 == value("OMNI_DTYPE_F32")
    assert N.DTYPE_BF16 == value("OMNI_DTYPE_BF16")
    assert N.DTYPE_FP8_E4M3 == value("OMNI_DTYPE_FP8_E4M3")
    assert N.DTYPE_I64 == value("OMNI_DTYPE_I64")
    assert N.ACT_SNAKE == value("OMNI_ACTIVATION_SNAKE")
    assert N.ACT_CLAMP == value("OMNI_ACTIVATION_CLAMP")
    assert N.RVQ_CLAMP == value("OMNI_RVQ_CLAMP")


def test_library_carries_gfx950_code_objects():
    # the offload bundle of every kernel names its target, amdgcn-amd-amdhsa--gfx950
    blob = N.LIB_PATH.read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    assert b"gfx942" not in blob and b"gfx90a" not in blob


def test_channel_embedding_tables_refuse_host_tables():
    """The fused MOSS-TTS channel sum runs on the GPU only: host tables are refused (the caller
    keeps its eager loop), and embed() before a successful refresh raises instead of computing."""
    import torch

    from sglang_omni_amd.kernels.channel_embedding import ChannelEmbeddingTables

    tables = ChannelEmbeddingTables()
    weights = [torch.zeros(4, 8, dtype=torch.bfloat16) for _ in range(3)]
    assert not tables.refresh(weights)
    assert tables._table_info is None
    try:
        tables.embed(torch.zeros(2, 3, dtype=torch.int64), weights)
    except N.OmniCodecError:
        pass
    else:
        raise AssertionError("embed without a refreshed table set must raise")
    assert tables.embed(torch.zeros(0, 3, dtype=torch.int64), weights).shape == (0, 8)
