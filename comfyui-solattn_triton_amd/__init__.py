"""Sol-Attn as a ComfyUI attention override, on MI355X (gfx950) HIP kernels.

A drop-in for kijai/ComfyUI-SolAttn_triton (/root/reference/__init__.py): the
"Patch Sol-Attn" node installs an ``optimized_attention_override`` on the model
(per-model, with the sigma window for dense warm-up steps), "Sol-Attn Block
Probe" measures per-block error, ``attention_sol`` is registered as
"sol_attn", and ``SOL_ATTN=1`` installs a global override for CLI runs.

The kernel-level API (``sol_attn``, ``sol_attn_int8``, ``prepare``,
``fused_preprocess``, ``quantize_bthd``, ``quantize_v_per_channel``,
``morton_perm``) lives in the submodules and needs no ComfyUI; the node layer
below is defined when ComfyUI is importable.
"""

import logging
import os

from ._dispatch import (  # noqa: F401  (re-exported API)
    BLOCK_SIZE,
    HEAD_DIM,
    MIN_TOKENS,
    _IMPORT_ERROR,
    _INT8_IMPORT_ERROR,
    _compose_module_patch,
    _ineligible,
    _install_block_index,
    _install_compose_hooks,
    _probe,
    _run,
    _sink_blocks,
    _sol_attn_int8_kernel,
    _sol_attn_kernel,
    _stats,
    log_probe_summary,
    make_override,
    make_probe_override,
    parse_blocks,
    parse_tau_profile,
    reset_sol_attn_stats,
    sol_attn_stats,
    try_sparse_default,
)

try:
    from comfy.ldm.modules.attention import attention_pytorch, register_attention_function, wrap_attn
    from comfy.patcher_extension import CallbacksMP
    from comfy_api.latest import ComfyExtension, io
    _COMFY_ERROR = None
except ImportError as exc:  # used outside ComfyUI: kernels only
    _COMFY_ERROR = exc

_BLOCK_CHOICES = ["64", "128"]


if _COMFY_ERROR is None:

    def _require_kernels(int8_qk):
        if _sol_attn_kernel is None:
            raise RuntimeError(f"Sol-Attn kernel unavailable: {_IMPORT_ERROR}")
        if int8_qk and _sol_attn_int8_kernel is None:
            raise RuntimeError(f"Sol-Attn INT8 kernel unavailable: {_INT8_IMPORT_ERROR}")

    def _model_family(diffusion_model):
        """'h3' (MiniMax-H3: rope_freqs + _forward), 'wan' (rope_encode + blocks) or None."""
        if hasattr(diffusion_model, "rope_freqs") and hasattr(diffusion_model, "_forward"):
            return "h3"
        if hasattr(diffusion_model, "rope_encode") and hasattr(diffusion_model, "blocks"):
            return "wan"
        return None

    def _install_reordering(diffusion_model, morton, sink_conditioning, block):
        """Install the model's reorder hooks; True when tokens will be reordered.
        H3's hooks also publish the video span the conditioning sink needs, so
        they go in whenever the sink is on, reordering or not."""
        family = _model_family(diffusion_model)
        if family == "h3" and (morton or sink_conditioning != "off"):
            from ._morton_h3 import install_h3_hooks
            install_h3_hooks(diffusion_model, block=block)
            return bool(morton)
        if family == "wan" and morton:
            from ._morton import install_wan_morton
            install_wan_morton(diffusion_model)
            return True
        if morton:
            logging.warning(f"[sol_attn] Morton reordering skipped: "
                            f"{type(diffusion_model).__name__} is neither Wan-style nor "
                            "MiniMax-H3. Sol-Attn itself still applies.")
        return False

    def _depth_controls(diffusion_model, dense_blocks, tau_profile, tau):
        """(dense block set, {block: tau}) for this model, with the block-index
        publisher installed when either is used."""
        blocks = getattr(diffusion_model, "blocks", None)
        count = 0 if blocks is None else len(blocks)
        dense = parse_blocks(dense_blocks, count)
        profile = parse_tau_profile(tau_profile or "", count)
        if not (dense or profile):
            return dense, profile
        if not _install_block_index(diffusion_model):
            logging.warning(f"[sol_attn] dense_blocks/tau_profile ignored: "
                            f"{type(diffusion_model).__name__} has no .blocks list to index")
            return frozenset(), {}
        if dense:
            logging.info(f"[sol_attn] keeping blocks {sorted(dense)} dense of {count}")
        if profile:
            by_level = {}
            for index, level in profile.items():
                by_level[level] = by_level.get(level, 0) + 1
            summary = ", ".join(f"{level} on {n} block(s)" for level, n in sorted(by_level.items()))
            logging.info(f"[sol_attn] per-block tau: {summary}; base {tau} elsewhere")
        return dense, profile

    def _is_self_attention_forward(key):
        """Object-patch keys like 'diffusion_model.blocks.3.self_attn.forward'."""
        if not key.endswith(".forward"):
            return False
        owner = key.rsplit(".", 2)[-2].lower()
        return "attn" in owner and "cross" not in owner and owner != "attn2"

    def _compose_object_patches(patched, diffusion_model):
        """Gate every object-patched self-attention forward on the clone, and
        hook the blocks so patches applied after this node compose too."""
        keys = []
        for key, forward in list(patched.object_patches.items()):
            if not _is_self_attention_forward(key) or getattr(forward, "_uses_optimized_attention", False):
                continue
            module = patched.get_model_object(key[: -len(".forward")])
            patched.add_object_patch(key, _compose_module_patch(module, forward))
            keys.append(key)
        if keys:
            logging.info(f"[sol_attn] composed with {len(keys)} object-patched attention "
                         f"forward(s) (e.g. {keys[0]})")
        family = _model_family(diffusion_model)
        if family is not None:
            _install_compose_hooks(diffusion_model, "attn" if family == "h3" else "self_attn")

    class SolAttnPatch(io.ComfyNode):
        """The "Patch Sol-Attn" node (/root/reference/__init__.py:422-606)."""

        @classmethod
        def define_schema(cls):
            return io.Schema(
                node_id="SolAttnPatch",
                display_name="Patch Sol-Attn",
                is_experimental=True,
                category="sol_attn",
                description="Sparsify self-attention with Sol-Attn (arXiv 2607.24027), with "
                            "optional Morton token reordering, INT8 QK, and an exact-KV sink "
                            "for MiniMax-H3's packed conditioning rows. bf16 + head_dim 128 "
                            "only; everything else falls back to the existing attention backend. "
                            "Runs on gfx950 (MI355X) HIP kernels.",
                inputs=[
                    io.Model.Input("model"),
                    io.Float.Input("tau", default=1.3, min=0.0, max=4.0, step=0.05,
                                   tooltip="Threshold beta. Higher is sparser: 1.0 ~ 16% of "
                                           "blocks kept exact, 1.5 ~ 7%, 2.0 ~ 2.7%."),
                    io.Float.Input("start_percent", default=0.2, min=0.0, max=1.0, step=0.01,
                                   tooltip="Run dense before this point. The paper uses 0.2."),
                    io.Float.Input("end_percent", default=0.9, min=0.0, max=1.0, step=0.01),
                    io.Int.Input("min_tokens", default=MIN_TOKENS, min=0, max=1 << 20, step=512,
                                 tooltip="Sequences shorter than this stay dense. On MI355X "
                                         "the sparse path already beats dense SDPA from 2048 "
                                         "tokens; lower this to trade exactness for speed."),
                    io.Boolean.Input("int8_qk", default=True,
                                     tooltip="INT8 QK in the exact branch (smoothed K, per-token "
                                             "scales) on the int8 matrix cores."),
                    io.Combo.Input("sink_conditioning",
                                   options=["exact_kv", "exact_kv_and_rows", "off"],
                                   default="exact_kv_and_rows",
                                   tooltip="MiniMax-H3 only. exact_kv: every query sees the packed "
                                           "text/audio/reference rows exactly. exact_kv_and_rows: "
                                           "also runs those query rows dense. No effect on other "
                                           "models."),
                    io.Boolean.Input("morton", default=False,
                                     tooltip="Reorder video tokens into Morton (Z-order) so each "
                                             "block is a compact 3D neighbourhood. Exactly neutral "
                                             "for dense attention. Wan and MiniMax-H3 only."),
                    io.Combo.Input("morton_curve", options=["3d", "2d_frame"], default="2d_frame",
                                   tooltip="3d interleaves t/h/w equally. 2d_frame Z-orders within "
                                           "each frame and keeps frame order."),
                    io.Boolean.Input("int8_pv", default=True,
                                     tooltip="Also run the exact branch's P@V in INT8 (per-row P "
                                             "scale, per-channel V scale). Only with int8_qk."),
                    io.Boolean.Input("verbose", default=False),
                    io.Boolean.Input("use_tma", default=False,
                                     tooltip="Accepted for workflow compatibility; there are no "
                                             "TMA descriptor kernels on this GPU, so it is ignored."),
                    io.String.Input("tau_profile", optional=True, force_input=True,
                                    tooltip="Per-block tau overriding the base value: 'blocks=tau' "
                                            "entries separated by ';' or newlines, '#' comments, "
                                            "e.g. '0-30=2.0' then '39-42=0.9'."),
                    io.String.Input("dense_blocks", default="",
                                    tooltip="Transformer blocks to keep dense, e.g. '0-2,-1'. "
                                            "Negative indices count from the end. Empty means "
                                            "sparsify all."),
                    io.Combo.Input("block_size", options=_BLOCK_CHOICES, default="64", optional=True,
                                   tooltip="Routing block in tokens. 64 is the reference's; 128 "
                                           "halves the pooled branch and suits long video."),
                    io.Combo.Input("int8_pv_codes", options=["block", "running"], default="block",
                                   optional=True,
                                   tooltip="With int8_pv: quantise P against each routed block's "
                                           "max (the reference's) or against the row's running "
                                           "max (int32 sums across blocks: a faster INT8 "
                                           "forward, coarser codes for blocks below the max)."),
                ],
                outputs=[io.Model.Output()],
            )

        @classmethod
        def execute(cls, model, tau, start_percent, end_percent, min_tokens, int8_qk,
                    sink_conditioning, morton, morton_curve, dense_blocks, verbose,
                    tau_profile=None, use_tma=False, int8_pv=True, block_size="64",
                    int8_pv_codes="block") -> io.NodeOutput:
            _require_kernels(int8_qk)
            block = int(block_size)
            diffusion_model = model.get_model_object("diffusion_model")
            reorder = _install_reordering(diffusion_model, morton, sink_conditioning, block)
            dense, profile = _depth_controls(diffusion_model, dense_blocks, tau_profile, tau)
            sampling = model.get_model_object("model_sampling")
            window = (float(sampling.percent_to_sigma(start_percent)),
                      float(sampling.percent_to_sigma(end_percent)))

            patched = model.clone()
            options = patched.model_options["transformer_options"]
            previous = options.get("optimized_attention_override")
            if previous is not None:
                logging.info("[sol_attn] chaining onto an existing attention override; Sol-Attn "
                             "takes first refusal and delegates everything else to it")
            _compose_object_patches(patched, diffusion_model)
            options["sol_compose"] = {"sigma_start": window[0], "sigma_end": window[1],
                                      "min_tokens": min_tokens}
            options["optimized_attention_override"] = make_override(
                tau=tau, min_tokens=min_tokens, sigma_start=window[0], sigma_end=window[1],
                verbose=verbose, int8_qk=int8_qk, sink_conditioning=sink_conditioning,
                use_tma=use_tma, dense_blocks=dense, tau_profile=profile, int8_pv=int8_pv,
                previous=previous, block=block, pv_codes=int8_pv_codes)
            options["sol_block_size"] = block
            if reorder:
                options.update(sol_morton=True, sol_morton_curve=morton_curve)
            reset_sol_attn_stats()
            return io.NodeOutput(patched)

    class SolAttnBlockProbe(io.ComfyNode):
        """Diagnostic node (/root/reference/__init__.py:609-646)."""

        @classmethod
        def define_schema(cls):
            return io.Schema(
                node_id="SolAttnBlockProbe",
                display_name="Sol-Attn Block Probe",
                is_experimental=True,
                category="sol_attn",
                description="Diagnostic. Place after Patch Sol-Attn: every attention call is "
                            "computed both sparse and dense, and each block's relative error "
                            "is logged worst-first when sampling ends. The image this produces "
                            "is the dense reference; remove the node once you have the numbers.",
                inputs=[io.Model.Input("model")],
                outputs=[io.Model.Output()],
            )

        @classmethod
        def execute(cls, model) -> io.NodeOutput:
            probed = model.clone()
            options = probed.model_options["transformer_options"]
            inner = options.get("optimized_attention_override")
            if inner is None:
                raise RuntimeError("Sol-Attn Block Probe needs an attention override to measure; "
                                   "connect it after Patch Sol-Attn.")
            diffusion_model = probed.get_model_object("diffusion_model")
            if not _install_block_index(diffusion_model):
                logging.warning(f"[sol_attn] probe: {type(diffusion_model).__name__} has no "
                                ".blocks list, so every error lands under block 'None'")
            options["optimized_attention_override"] = make_probe_override(inner)
            _probe.clear()
            probed.add_callback(CallbacksMP.ON_CLEANUP, log_probe_summary)
            return io.NodeOutput(probed)

    @wrap_attn
    def attention_sol(q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                      skip_output_reshape=False, **kwargs):
        """The "sol_attn" registry entry: the sparse path with the registry
        defaults (tau 1.0, MIN_TOKENS tokens, BF16, no sigma window), ComfyUI's
        PyTorch attention otherwise (/root/reference/__init__.py:649-663)."""
        out = try_sparse_default(q, k, v, heads, mask, skip_reshape, skip_output_reshape,
                                 kwargs.get("scale"))
        if out is not None:
            return out
        return attention_pytorch(q, k, v, heads, mask=mask, skip_reshape=skip_reshape,
                                 skip_output_reshape=skip_output_reshape, **kwargs)

    register_attention_function("sol_attn", attention_sol)

    def _install_global_override(environ=os.environ):
        """SOL_ATTN set (not '0', '' or 'false'): route every optimized
        attention call through attention_sol, for CLI runs without the node."""
        if environ.get("SOL_ATTN", "0") in ("0", "", "false"):
            return False
        if _sol_attn_kernel is None:
            logging.error(f"[sol_attn] SOL_ATTN set but kernel import failed: {_IMPORT_ERROR}")
            return False
        import comfy.ldm.modules.attention as attention_module
        attention_module.optimized_attention = attention_sol
        attention_module.optimized_attention_masked = attention_sol
        logging.info("[sol_attn] global override active (node patch is preferred)")
        return True

    _install_global_override()

    class SolAttnExtension(ComfyExtension):
        async def get_node_list(self):
            return [SolAttnPatch, SolAttnBlockProbe]

    async def comfy_entrypoint() -> SolAttnExtension:
        return SolAttnExtension()
