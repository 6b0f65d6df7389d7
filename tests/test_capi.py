"""The C-ABI library: loads, exports every entry point declared in
include/infengine.h, and rejects bad arguments on the host before any GPU work
(the reference's launchers had no argument checks at all).  CPU only: no call
here reaches the GPU.
"""
import ctypes as C
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "infengine.h"

IE_ERR_INVALID_ARG = -1


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"IE_API\s+[\w\s\*]+?\b(ie_\w+)\s*\(", text)))


def test_header_declares_the_engine_boundary():
    syms = declared_symbols()
    for name in ("ie_prefill", "ie_decode_step", "ie_model_weights_random_init",
                 "ie_kv_cache_size", "ie_attn_workspace_size", "ie_ffn_workspace_size",
                 "ie_multiply_by_weight", "ie_decode_attn", "ie_attn", "ie_ffn", "ie_rmsnorm",
                 "ie_apply_rope", "ie_emblookup", "ie_lm_head", "ie_sample_token_amax",
                 "ie_residual_add", "ie_swiglu", "ie_scale_causal_softmax", "ie_init_rope_buffer"):
        assert name in syms, name


def test_library_exports_every_declared_symbol(hip):
    lib = C.CDLL(str(hip.LIB_PATH))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_ctypes_signatures_cover_the_header(hip):
    from infengine_amd._lib import SIGNATURES
    assert sorted(SIGNATURES) == declared_symbols()


def test_model_weights_struct_layout_matches_header(hip, tmp_path):
    """The ctypes mirror has the C compiler's size and offsets of ie_model_weights."""
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "infengine.h"\n'
                   'int main(void) { printf("%zu %zu %zu %zu %zu\\n", sizeof(ie_model_weights), '
                   'offsetof(ie_model_weights, layers), offsetof(ie_model_weights, rope), '
                   'offsetof(ie_model_weights, storage), offsetof(ie_model_weights, rope_rows)); '
                   'return 0; }\n')
    exe = tmp_path / "layout"
    import pathlib
    import subprocess
    inc = pathlib.Path(__file__).resolve().parent.parent / "include"
    subprocess.run(["gcc", f"-I{inc}", str(src), "-o", str(exe)], check=True)
    want = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True,
                                           check=True).stdout.split()]
    S = hip.ModelWeightsStruct
    assert [C.sizeof(S), S.layers.offset, S.rope.offset, S.storage.offset,
            S.rope_rows.offset] == want
    # emb + 32 layers x 9 pointers + final_norm + lm_head + rope(2) + storage, then rope_rows
    assert want[4] == 8 * (1 + 32 * 9 + 2 + 2 + 1)


def test_sizes(hip):
    lib = hip.lib
    assert lib.ie_kv_cache_size() == 32 * 2 * 8 * 8192 * 128 * 2      # attn.cu:304-307
    S = 2048
    assert lib.ie_attn_workspace_size(S) >= S * 6144 * 2 + S * 4096 * 2
    assert lib.ie_ffn_workspace_size(S) >= S * 14336 * 2
    # decode needs a fixed amount, so a small-S workspace still serves long decodes
    assert lib.ie_attn_workspace_size(1) == lib.ie_attn_workspace_size(0)
    # top-p: the fp32 exponentials, then per-row state (< 128 KiB a row)
    assert 16 * 128256 * 4 < lib.ie_top_p_workspace_size(16, 128256) <= 16 * 128256 * 4 + 16 * (128 << 10)
    assert lib.ie_top_p_workspace_size(1, 128256) < lib.ie_top_p_workspace_size(2, 128256)


BOGUS = C.c_void_p(0x1000)   # never dereferenced: every call below fails validation first


@pytest.mark.parametrize("call", [
    lambda l: l.ie_context_create(None, 0, None),
    lambda l: l.ie_decode_step(None, None, 1, *[BOGUS] * 8),
    lambda l: l.ie_prefill(None, None, 1, *[BOGUS] * 8),
    lambda l: l.ie_multiply_by_weight(None, 1, 4096, 4096, BOGUS, BOGUS, BOGUS),
    lambda l: l.ie_emblookup(4, None, BOGUS, BOGUS, None),
    lambda l: l.ie_rmsnorm(4, BOGUS, None, BOGUS, None),
    lambda l: l.ie_residual_add(-1, 4096, BOGUS, BOGUS, None),
    lambda l: l.ie_apply_rope(8190, 8, 4, BOGUS, BOGUS, BOGUS, BOGUS, 1, None),
    lambda l: l.ie_scale_causal_softmax(0, BOGUS, BOGUS, 0, None),
    lambda l: l.ie_model_weights_free(None),
    lambda l: l.ie_sample_top_p(None, 1, 128256, BOGUS, 0.7, 0.9, 1, 0, BOGUS, BOGUS),
    lambda l: l.ie_sample_top_p_noalloc(None, 17, 131072, BOGUS, 0.7, 0.9, 1, 0, BOGUS),
    lambda l: l.ie_prefill_paged_chunk(None, None, 0, 1, *[BOGUS] * 8, 1, BOGUS),
    lambda l: l.ie_attn_prefill_core_paged(None, 1, 9000, BOGUS, BOGUS, 1, BOGUS, 0, BOGUS),
    lambda l: l.ie_decoder_layer_decode(None, None, 0, 1, BOGUS, BOGUS, BOGUS, BOGUS),
    lambda l: l.ie_decoder_layer_prefill(None, None, 0, 1, *[BOGUS] * 5),
    lambda l: l.ie_decoder_layer_prefill_last_row(None, None, 0, 1, *[BOGUS] * 5),
    lambda l: l.ie_decoder_layer_batched(None, None, 0, 1, None, *[BOGUS] * 4),
])
def test_host_side_validation(hip, call):
    assert call(hip.lib) == IE_ERR_INVALID_ARG
    assert hip.last_error()          # a message explains the rejection


def test_error_raises_with_message(hip):
    with pytest.raises(hip.IEError, match="rope"):
        hip.check(hip.lib.ie_apply_rope(8190, 8, 4, BOGUS, BOGUS, BOGUS, BOGUS, 1, None))
