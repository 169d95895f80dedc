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
                    io.Int.Input("min_tokens", default=4096, min=0, max=1 << 20, step=512,
                                 tooltip="Sequences shorter than this stay dense."),
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
                ],
                outputs=[io.Model.Output()],
            )

        @classmethod
        def execute(cls, model, tau, start_percent, end_percent, min_tokens, int8_qk,
                    sink_conditioning, morton, morton_curve, dense_blocks, verbose,
                    tau_profile=None, use_tma=False, int8_pv=True, block_size="64") -> io.NodeOutput:
            if _sol_attn_kernel is None:
                raise RuntimeError(f"Sol-Attn kernel unavailable: {_IMPORT_ERROR}")
            if int8_qk and _sol_attn_int8_kernel is None:
                raise RuntimeError(f"Sol-Attn INT8 kernel unavailable: {_INT8_IMPORT_ERROR}")
            block = int(block_size)

            diffusion_model = model.get_model_object("diffusion_model")
            is_h3 = hasattr(diffusion_model, "rope_freqs") and hasattr(diffusion_model, "_forward")
            is_wan = hasattr(diffusion_model, "rope_encode") and hasattr(diffusion_model, "blocks")

            # H3 publishes its segment layout from the same hooks Morton uses, so
            # the conditioning sink needs them even when reordering is off.
            reorder = False
            if is_h3 and (morton or sink_conditioning != "off"):
                from ._morton_h3 import install_h3_hooks
                install_h3_hooks(diffusion_model, block=block)
                reorder = morton
            elif is_wan and morton:
                from ._morton import install_wan_morton
                install_wan_morton(diffusion_model)
                reorder = True
            elif morton:
                logging.warning(f"[sol_attn] Morton reordering skipped: "
                                f"{type(diffusion_model).__name__} is neither Wan-style nor "
                                "MiniMax-H3. Sol-Attn itself still applies.")

            blocks = getattr(diffusion_model, "blocks", None)
            count = len(blocks) if blocks is not None else 0
            dense = parse_blocks(dense_blocks, count)
            profile = parse_tau_profile(tau_profile or "", count)
            if (dense or profile) and not _install_block_index(diffusion_model):
                logging.warning(f"[sol_attn] dense_blocks/tau_profile ignored: "
                                f"{type(diffusion_model).__name__} has no .blocks list to index")
                dense, profile = frozenset(), {}
            if dense:
                logging.info(f"[sol_attn] keeping blocks {sorted(dense)} dense of {count}")
            if profile:
                levels = {}
                for blk, level in sorted(profile.items()):
                    levels.setdefault(level, []).append(blk)
                logging.info("[sol_attn] per-block tau: "
                             + ", ".join(f"{lv} on {len(bs)} block(s)" for lv, bs in sorted(levels.items()))
                             + f"; base {tau} elsewhere")

            model_sampling = model.get_model_object("model_sampling")
            sigma_start = float(model_sampling.percent_to_sigma(start_percent))
            sigma_end = float(model_sampling.percent_to_sigma(end_percent))

            m = model.clone()
            options = m.model_options["transformer_options"]
            previous = options.get("optimized_attention_override")
            if previous is not None:
                logging.info("[sol_attn] chaining onto an existing attention override; Sol-Attn "
                             "takes first refusal and delegates everything else to it")

            # Forward-level patches bypass optimized_attention; gate each one.
            composed = []
            for key, patched in list(m.object_patches.items()):
                if not key.endswith(".forward"):
                    continue
                owner = key.rsplit(".", 2)[-2].lower()
                if "attn" not in owner or "cross" in owner or owner == "attn2":
                    continue
                if getattr(patched, "_uses_optimized_attention", False):
                    continue
                module = m.get_model_object(key[: -len(".forward")])
                m.add_object_patch(key, _compose_module_patch(module, patched))
                composed.append(key)
            if composed:
                logging.info(f"[sol_attn] composed with {len(composed)} object-patched attention "
                             f"forward(s) (e.g. {composed[0]})")
            if is_h3:
                _install_compose_hooks(diffusion_model, "attn")
            elif is_wan:
                _install_compose_hooks(diffusion_model, "self_attn")

            options["sol_compose"] = {"sigma_start": sigma_start, "sigma_end": sigma_end,
                                      "min_tokens": min_tokens}
            options["optimized_attention_override"] = make_override(
                tau=tau, min_tokens=min_tokens, sigma_start=sigma_start, sigma_end=sigma_end,
                verbose=verbose, int8_qk=int8_qk, sink_conditioning=sink_conditioning,
                use_tma=use_tma, dense_blocks=dense, tau_profile=profile, int8_pv=int8_pv,
                previous=previous, block=block)
            options["sol_block_size"] = block
            if reorder:
                options["sol_morton"] = True
                options["sol_morton_curve"] = morton_curve
            reset_sol_attn_stats()
            return io.NodeOutput(m)

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
            m = model.clone()
            inner = m.model_options["transformer_options"].get("optimized_attention_override")
            if inner is None:
                raise RuntimeError("Sol-Attn Block Probe needs an attention override to measure; "
                                   "connect it after Patch Sol-Attn.")
            diffusion_model = m.get_model_object("diffusion_model")
            if not _install_block_index(diffusion_model):
                logging.warning(f"[sol_attn] probe: {type(diffusion_model).__name__} has no "
                                ".blocks list, so every error lands under block 'None'")
            m.model_options["transformer_options"]["optimized_attention_override"] = \
                make_probe_override(inner)
            _probe.clear()
            m.add_callback(CallbacksMP.ON_CLEANUP, log_probe_summary)
            return io.NodeOutput(m)

    @wrap_attn
    def attention_sol(q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                      skip_output_reshape=False, **kwargs):
        """Registry entry point with the defaults (tau 1.0, min_tokens 4096, bf16,
        no sigma window); /root/reference/__init__.py:649-663."""
        if mask is None:
            try:
                out = _run(q, k, v, heads, skip_reshape, skip_output_reshape,
                           kwargs.get("scale", None), 1.0, 4096, False)
                if out is not None:
                    return out
            except Exception as exc:
                _stats["errors"] += 1
                from ._dispatch import _log_kernel_failure
                _log_kernel_failure(exc)
        return attention_pytorch(q, k, v, heads, mask=mask, skip_reshape=skip_reshape,
                                 skip_output_reshape=skip_output_reshape, **kwargs)

    register_attention_function("sol_attn", attention_sol)

    if os.environ.get("SOL_ATTN", "0") not in ("0", "", "false"):
        if _sol_attn_kernel is None:
            logging.error(f"[sol_attn] SOL_ATTN set but kernel import failed: {_IMPORT_ERROR}")
        else:
            import comfy.ldm.modules.attention as _attn_mod

            _attn_mod.optimized_attention = attention_sol
            _attn_mod.optimized_attention_masked = attention_sol
            logging.info("[sol_attn] global override active (node patch is preferred)")

    class SolAttnExtension(ComfyExtension):
        async def get_node_list(self):
            return [SolAttnPatch, SolAttnBlockProbe]

    async def comfy_entrypoint() -> SolAttnExtension:
        return SolAttnExtension()
