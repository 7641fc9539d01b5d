"""The C-ABI entry points as PyTorch operators: ``torch.ops.fast_mimi_amd.*``.

Each stream-taking ``fm_*`` function of ``include/fast_mimi_amd.h`` is
registered (library ``fast_mimi_amd``, operator name without the ``fm_``
prefix) with a schema that mirrors its C signature: device pointers become
optional tensors (``const T*`` read-only, ``T*`` mutated in place; a residual input
shares the alias set of the output it may be added into in place), ints and
sizes become ``int``, floats ``float``.  The trailing ``hipStream_t`` is the
current torch stream of the calling device, so calls recorded under
``torch.cuda.graph`` land in the captured graph.  The operators return
nothing; a non-zero status raises ``NativeError``.  Every operator has a
fake (meta) implementation, so FX tracing and ``torch.compile`` see them as
opaque mutating calls.  The implementation is the HIP library itself; there
is no other backend.
"""

from __future__ import annotations

import torch

from . import _native as nat

# Argument kinds and names per entry point, in C order, stream excluded
# (in: const pointer, out: mutable pointer, res: const pointer that may be
# the same memory as the output ``y`` (the runtime adds a residual in place,
# y = residual + ...), i: integer / size, f: float).
SPECS = {
    "fm_split_weights": "in:weight_packed i:rows i:cols out:planes",
    "fm_conv1d": "in:x i:batch i:length i:in_channels in:weight_packed in:bias i:out_channels i:kernel i:stride i:pad_mode i:flags res:residual out:y i:y_length out:workspace i:workspace_bytes",
    "fm_conv1d_rows": "in:x i:batch i:length i:in_channels in:weight in:bias i:bias_len i:out_channels i:kernel i:stride i:pad_mode i:flags res:residual out:y",
    "fm_conv1d_valid": "in:x i:batch i:length i:in_channels in:weight_packed in:bias i:out_channels i:kernel i:stride i:flags res:residual out:y out:workspace i:workspace_bytes",
    "fm_conv_transpose1d": "in:x i:batch i:length i:in_channels in:weight_packed in:bias i:out_channels i:kernel i:stride i:flags res:residual out:y out:workspace i:workspace_bytes",
    "fm_linear": "in:x i:rows i:in_features in:weight_packed i:out_features i:flags res:residual in:scale out:y out:workspace i:workspace_bytes",
    "fm_linear_rope": "in:x i:rows i:in_features in:weight_packed i:out_features i:flags in:cos_table in:sin_table i:rope_cols i:rows_per_seq out:y out:workspace i:workspace_bytes",
    "fm_resblock": "in:x i:batch i:length i:channels in:w1_packed in:b1 in:w2_packed in:b2 i:elu_out out:y",
    "fm_conv_resblock64": "in:wav i:batch i:length in:w0_packed in:b0 in:w1_packed in:b1 in:w2_packed in:b2 i:elu_out out:y",
    "fm_resblock64_conv": "in:x i:batch i:length in:w1_packed in:b1 in:w2_packed in:b2 i:elu_mid in:w3_packed in:b3 i:y_len out:out out:workspace i:workspace_bytes",
    "fm_row_linear": "in:x i:rows i:in_features in:ln_gamma in:ln_beta f:ln_eps in:weight i:out_features i:flags res:residual in:scale in:rope_cos in:rope_sin i:rope_cols i:rows_per_seq out:y",
    "fm_row_linear_packed": "in:x i:rows i:in_features in:ln_gamma in:ln_beta f:ln_eps in:weight_packed i:out_features i:flags res:residual in:scale in:rope_cos in:rope_sin i:rope_cols i:rows_per_seq out:y",
    "fm_pack_row_weights": "in:weight i:out_features i:in_features out:out",
    "fm_row_linear_packed_upsample": "in:x i:rows i:in_features in:weight_packed i:out_features i:rows_per_seq in:up_weight out:y",
    "fm_apply_rope": "out:x i:rows i:ld i:rope_cols i:head_dim in:cos_table in:sin_table i:rows_per_seq",
    "fm_layer_norm": "in:x in:gamma in:beta i:rows i:channels f:eps out:y",
    "fm_window_attention": "in:qkv i:ld_qkv i:q_offset i:k_offset i:v_offset in:cos_table in:sin_table i:batch i:length i:heads i:kv_heads i:head_dim i:window f:scale out:out i:ld_out",
    "fm_window_attention_rows": "in:qkv i:ld_qkv i:q_offset i:k_offset i:v_offset in:cos_table in:sin_table i:batch i:length i:query_start i:heads i:kv_heads i:head_dim i:window f:scale out:out i:ld_out",
    "fm_rvq_prepare_codebook": "in:embed_sum in:cluster_usage i:entries i:dim f:eps out:embed out:embed_t out:norms",
    "fm_rvq_encode": "in:x i:ld_x i:rows i:rows_per_batch i:dim i:entries i:count in:embeds in:embeds_t in:norms out:codes i:batch_stride out:workspace i:workspace_bytes",
    "fm_rvq_encode_split": "in:x i:ld_x i:rows i:rows_per_batch i:dim i:entries i:n_semantic i:n_acoustic in:embeds in:embeds_t in:norms out:codes i:batch_stride out:workspace i:workspace_bytes",
    "fm_rvq_encode_split_noalloc": "in:x i:ld_x i:rows i:rows_per_batch i:dim i:entries i:n_semantic i:n_acoustic in:embeds in:embeds_t in:norms out:codes i:batch_stride",
    "fm_rvq_decode": "in:codes i:batch i:num_codebooks i:frames i:num_semantic in:embeds i:entries i:dim out:out",
    "fm_upsample_depthwise": "in:x i:batch i:length i:channels in:weight i:kernel i:stride out:y",
    "fm_copy_buffers": "in:src0 out:dst0 i:bytes0 in:src1 out:dst1 i:bytes1",
}

_TYPE = {"i": "int", "f": "float"}
_lib = torch.library.Library("fast_mimi_amd", "DEF")


def _schema(op: str, spec: str) -> str:
    items = [item.split(":") for item in spec.split()]
    # Alias set of each mutated pointer; a ``res`` input shares the set of the
    # output ``y``, so functionalization sees that y may overwrite it.
    sets = {name: f"a{i}" for i, name in enumerate(n for k, n in items if k == "out")}
    args = []
    for kind, name in items:
        if kind == "in":
            args.append(f"Tensor? {name}")
        elif kind == "res":
            args.append(f"Tensor({sets['y']})? {name}")
        elif kind == "out":
            args.append(f"Tensor({sets[name]}!)? {name}")
        else:
            args.append(f"{_TYPE[kind]} {name}")
    return f"{op}({', '.join(args)}) -> ()"


def _make_impl(entry: str, pointer_args: tuple[int, ...]):
    def impl(*args):
        device = next((a.device for a in args if isinstance(a, torch.Tensor)), None)
        stream = torch.cuda.current_stream(device).cuda_stream
        values = list(args)
        for i in pointer_args:
            values[i] = None if values[i] is None else values[i].data_ptr()
        nat.call(entry, *values, stream)

    return impl


def _fake(*args):
    return None


for _entry, _spec in SPECS.items():
    _op = _entry[3:]
    _lib.define(_schema(_op, _spec))
    _ptrs = tuple(i for i, item in enumerate(_spec.split()) if item.split(":")[0] in ("in", "res", "out"))
    _lib.impl(_op, _make_impl(_entry, _ptrs), "CompositeExplicitAutograd")
    torch.library.register_fake(f"fast_mimi_amd::{_op}", _fake, lib=_lib)


def op(entry: str):
    """The operator of C-ABI entry point ``entry`` (e.g. ``"fm_conv1d"``)."""
    return getattr(torch.ops.fast_mimi_amd, entry[3:])


def call(entry: str, *args) -> None:
    """Run C-ABI entry point ``entry`` through its operator."""
    getattr(torch.ops.fast_mimi_amd, entry[3:])(*args)
