"""CPU: the C-ABI library loads and exports exactly what include/dmoe.h
declares, the ctypes mirror matches the C struct layouts, and the entry
points reject bad arguments without touching a GPU."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "dmoe.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dmoe_[a-z0-9_]+)\s*\(", text)))


def test_exports_match_header():
    import dmoe
    lib = dmoe.load()
    names = _declared()
    assert len(names) >= 14
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(dmoe.EXPORTS) == names
    out = subprocess.run(["nm", "-D", "--defined-only", str(dmoe.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = sorted(set(re.findall(r" T (dmoe_[a-z0-9_]+)$", out, flags=re.M)))
    assert exported == names


def test_struct_layouts_match_c(tmp_path):
    from dmoe import _abi
    src = tmp_path / "probe.c"
    src.write_text(f"""
#include <stdio.h>
#include <stddef.h>
#include "{HEADER}"
int main(void) {{
  printf("%zu %zu %zu %zu\\n", sizeof(dmoe_tensor), sizeof(dmoe_hparams),
         sizeof(dmoe_layer_desc), sizeof(dmoe_debug));
  printf("%zu %zu %zu\\n", offsetof(dmoe_tensor, ne), offsetof(dmoe_tensor, nb),
         offsetof(dmoe_hparams, routed_scaling));
  printf("%zu %zu\\n", offsetof(dmoe_layer_desc, exp_down), offsetof(dmoe_debug, perm));
  printf("%d\\n", DMOE_N_STAGES);
  return 0;
}}""")
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-o", str(exe), str(src)], check=True)
    vals = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True,
                                           check=True).stdout.split()]
    mine = [C.sizeof(_abi.Tensor), C.sizeof(_abi.HParams), C.sizeof(_abi.LayerDesc),
            C.sizeof(_abi.Debug), _abi.Tensor.ne.offset, _abi.Tensor.nb.offset,
            _abi.HParams.routed_scaling.offset, _abi.LayerDesc.exp_down.offset,
            _abi.Debug.perm.offset]
    import dmoe
    assert vals == mine + [dmoe.N_STAGES]


def test_row_size_matches_oracle(O):
    import dmoe
    lib = dmoe.load()
    for t in (0, 1, 8, 12):
        for n in (256, 1024, 4096):
            assert lib.dmoe_row_size(t, n) == O.row_size(t, n)
    assert lib.dmoe_row_size(12, 100) == 0        # not a whole super-block
    assert lib.dmoe_row_size(2, 256) == 0         # unsupported type
    assert lib.dmoe_row_size(12, 4096) == 2304 and lib.dmoe_row_size(8, 4096) == 4352


def test_null_context_is_rejected():
    import dmoe
    from dmoe import _abi
    lib = dmoe.load()
    hp = dmoe.hparams_of(256, 16, 4, 8, 32)
    d = _abi.LayerDesc()
    out = C.c_void_p()
    E = _abi.ERR_INVALID_ARG
    assert lib.dmoe_create(0, None) == E
    assert lib.dmoe_layer_upload(None, C.byref(hp), C.byref(d), C.byref(out)) == E
    assert lib.dmoe_layer_wrap_device(None, C.byref(hp), C.byref(d), C.byref(out)) == E
    assert lib.dmoe_layer_forward(None, None, None, 32, None, None) == E
    assert lib.dmoe_layer_forward_device(None, None, None, 32, None, None) == E
    assert lib.dmoe_route_logits(None, C.byref(hp), None, None, 32, None) == E
    assert lib.dmoe_quantize_device(None, 12, None, None, 1, 256, None) == E
    assert lib.dmoe_residual_rmsnorm(None, None, None, None, None, 32, 4096, 1e-6, None) == E
    assert lib.dmoe_profile_enable(None, 1) == E
    assert lib.dmoe_profile_read(None, None, None) == E
    assert lib.dmoe_last_error(None) == b"null context"
    lib.dmoe_destroy(None)
    lib.dmoe_layer_free(None)
    assert lib.dmoe_layer_kernel_path(None) == -1
    from dmoe import gguf
    gguf._bind(lib)
    assert lib.dmoe_gguf_open(None, C.byref(out), None, 0) == E
    lib.dmoe_gguf_close(None)
    assert lib.dmoe_gguf_get_u32(None, b"expert_count", None) == E
    assert lib.dmoe_gguf_tensor_count(None) == -1
    assert lib.dmoe_gguf_tensor_name(None, 0) is None
    assert lib.dmoe_gguf_layer_desc(None, 0, None) == E
    assert lib.dmoe_dense_upload(None, 256, 256, None, None, None, C.byref(out)) == E
    names = [lib.dmoe_stage_name(i).decode() for i in range(dmoe.N_STAGES)]
    assert names[0] == "front" and "gateup_routed" in names
    assert lib.dmoe_stage_name(99) == b""
