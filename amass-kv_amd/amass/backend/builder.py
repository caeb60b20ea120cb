"""AMASS metadata builder: the platform's builder + the persistent AMASS decode state.

Reference: ``backend/builder.py:81-479`` (a FlashAttentionMetadataBuilder subclass).
Here it is a mixin placed in front of whichever metadata builder vLLM's ROCm platform
picked.  It owns the Stage-A lifecycle:

* the QuadState / R8State is allocated once, lazily at the first build() after the
  KV cache exists (it is sized by ``cache_config.num_gpu_blocks``), so every buffer
  address stays fixed across HIP-graph replays; at the same time the per-layer
  resident KV tensors are keyed ``data_ptr -> layer`` from the compilation config's
  static forward context (the tensor object the impl receives);
* summaries of newly finalised pages are (re)built outside the graph, in build():
  a steady batch rebuilds only the rows that crossed a page boundary (``*_build_tail``),
  the first build summarises everything (``*_build_bulk``) and later batch-composition
  changes rebuild only stale blocks (``*_build_delta``, tag-gated);
  cudagraph-capture dummy batches skip this;
* ``derive_page_params`` runs once per step (one launch), only on steps where
  ceil(seq_len / page) can have changed;
* the state is attached as ``md.amass`` for the impl;
* mem-v (reference builder.py:243-330, shadow): the Tier is allocated lazily like the
  state, and every step -- prefill and decode -- runs ``tier.begin_step`` outside the
  graph (invalidate the rewritten pages, flush complete staged pages to the pinned pool,
  allocate staging blocks, token slots) over the padded token count; the tier is attached
  as ``md.amass_tier`` (also on capture batches, where begin_step is skipped, so the
  captured forward contains the impl's V scatter).

With the HIP kernels the pure-decode pipeline is fixed-shape, allocation-free and
host-sync-free, so the builder declares UNIFORM_SINGLE_TOKEN_DECODE graph support
(reference builder.py:81-88) unless the config forces eager mode or this layer shape
is not served.
"""
from __future__ import annotations

import traceback

import torch

from . import _runtime

_NOTICE = set()


def _notice(msg: str) -> None:
    if msg not in _NOTICE:
        _NOTICE.add(msg)
        print(f"[amass] {msg}", flush=True)


def _cg_support():
    try:
        from vllm.v1.attention.backend import AttentionCGSupport
    except ImportError:                                     # older vLLM layouts
        from vllm.v1.attention.backends.utils import AttentionCGSupport
    return AttentionCGSupport


def _host_seq_lens(cam):
    """The runner's host copy of seq_lens without touching deprecated properties
    (reference builder.py:46-64 found the deprecated accessor costly per step)."""
    for name in ("seq_lens_cpu_upper_bound", "_seq_lens_cpu", "seq_lens_cpu"):
        sl = getattr(cam, name, None)
        if isinstance(sl, torch.Tensor):
            return sl
    return None


def _kv_tensor(mod):
    kvc = getattr(mod, "kv_cache", None) if mod is not None else None
    if isinstance(kvc, (list, tuple)):            # one cache per virtual engine
        kvc = kvc[0] if kvc else None
    return kvc if isinstance(kvc, torch.Tensor) and kvc.numel() > 0 else None


def _max_pages(vllm_config, block: int):
    """Pages of the longest sequence the engine admits (None if it does not say)."""
    mlen = getattr(getattr(vllm_config, "model_config", None), "max_model_len", None)
    return -(-int(mlen) // block) if isinstance(mlen, int) and mlen > 0 else None


def _geometry(vllm_config, kv_cache_spec):
    """(n_kv, G, head_size, block_size) of the layers this builder serves."""
    n_kv = int(kv_cache_spec.num_kv_heads)
    head = int(kv_cache_spec.head_size)
    block = int(kv_cache_spec.block_size)
    mc = vllm_config.model_config
    try:
        n_q = int(mc.get_num_attention_heads(vllm_config.parallel_config))
    except Exception:  # noqa: BLE001 - minimal configs in tests
        n_q = int(getattr(mc, "num_attention_heads", n_kv))
    return n_kv, max(n_q // n_kv, 1), head, block


class AmassMetadataBuilderMixin:
    """Mixed in front of the platform's metadata builder class."""

    @classmethod
    def get_cudagraph_support(cls, vllm_config, kv_cache_spec):
        cg = _cg_support()
        cfg = _runtime.get_config()
        n_kv, G, head, block = _geometry(vllm_config, kv_cache_spec)
        if (cfg is not None and cfg.variant == "fast" and not cfg.force_eager
                and _runtime.unsupported_reason(
                    cfg, head_size=head, block_size=block, G=G, n_kv=n_kv,
                    max_pages=_max_pages(vllm_config, block)) is None):
            return cg.UNIFORM_SINGLE_TOKEN_DECODE
        return cg.NEVER

    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        super().__init__(kv_cache_spec, layer_names, vllm_config, device)
        self._amass_cfg = _runtime.get_config()
        self._amass_device = device
        self._amass_vllm_config = vllm_config
        self._amass_layers = list(layer_names)
        self._amass_n_kv, self._amass_G, head, block = _geometry(vllm_config,
                                                                 kv_cache_spec)
        self._amass_state = None
        self._amass_tier = None
        self._amass_tier_tried = False
        self._amass_mem = self._amass_cfg is not None and self._amass_cfg.is_mem
        self._amass_layer_k = None
        self._amass_prev = None
        self._amass_built_once = False
        self._amass_capturing = False
        why = _runtime.unsupported_reason(self._amass_cfg, head_size=head,
                                          block_size=block, G=self._amass_G,
                                          n_kv=self._amass_n_kv,
                                          max_pages=_max_pages(vllm_config, block))
        self._amass_enabled = why is None
        if why is not None:
            _notice(f"stock attention kept: {why}")

    # ---- lazy state (num_gpu_blocks is known only once the cache is allocated) ------- #
    def _amass_layer_map(self):
        """(per-layer resident KV tensors, data_ptr -> layer), or None before binding."""
        sfc = self._amass_vllm_config.compilation_config.static_forward_context
        layer_kv, ptr2layer = [], {}
        for lidx, name in enumerate(self._amass_layers):
            kvc = _kv_tensor(sfc.get(name))
            if kvc is None:
                return None
            layer_kv.append(kvc)
            ptr2layer[kvc.data_ptr()] = lidx
        return layer_kv, ptr2layer

    def _amass_ensure_tier(self):
        if self._amass_tier is not None or self._amass_tier_tried or not self._amass_enabled:
            return self._amass_tier
        vc = self._amass_vllm_config
        nb = getattr(vc.cache_config, "num_gpu_blocks", None)
        bound = self._amass_layer_map() if nb else None
        if bound is None:
            return None                          # profiling run / not bound: retry
        self._amass_tier_tried = True
        layer_kv, ptr2layer = bound
        try:
            sched, comp = vc.scheduler_config, vc.compilation_config
            max_reqs = sched.max_num_seqs
            max_tokens = max(int(getattr(sched, "max_num_batched_tokens", 0) or 0),
                             int(getattr(comp, "max_cudagraph_capture_size", 0) or 0),
                             max_reqs) + 8
            tier = _runtime.make_tier(
                self._amass_cfg, self._amass_device, num_layers=len(self._amass_layers),
                num_blocks=int(nb), n_kv=self._amass_n_kv, max_reqs=max_reqs,
                max_pages=-(-vc.model_config.max_model_len // _runtime.PAGE),
                max_tokens=max_tokens, dtype=layer_kv[0].dtype)
            tier._layer_of = ptr2layer
            self._amass_tier = tier
            _notice(f"Tier allocated (mem-v shadow): {tier.bytes_report()}")
        except Exception as e:  # noqa: BLE001 - mem-v keeps the stock attention
            print("[amass] Tier allocation failed; stock attention kept:", flush=True)
            traceback.print_exception(type(e), e, e.__traceback__)
        return self._amass_tier

    def _amass_tier_step(self, md, cam):
        tier = self._amass_ensure_tier()
        if tier is None:
            return md
        if not self._amass_capturing:
            sm = getattr(md, "slot_mapping", None)
            n_tok = int(sm.shape[0]) if sm is not None else int(cam.num_actual_tokens)
            try:
                tier.begin_step(md.block_table, md.seq_lens, md.query_start_loc, n_tok)
            except Exception as e:  # noqa: BLE001
                print("[amass] tier.begin_step failed (this step keeps the stock "
                      "attention):", flush=True)
                traceback.print_exception(type(e), e, e.__traceback__)
                return md
        md.amass_tier = tier
        return md

    def _amass_ensure_state(self):
        if self._amass_state is not None or not self._amass_enabled:
            return self._amass_state
        vc = self._amass_vllm_config
        nb = getattr(vc.cache_config, "num_gpu_blocks", None)
        if not nb:
            return None
        bound = self._amass_layer_map()
        if bound is None:
            return None                          # not bound yet: retry next build
        layer_kv, ptr2layer = bound
        try:
            from ..attention.decode import _split_kv
            cfg = self._amass_cfg
            max_reqs = vc.scheduler_config.max_num_seqs
            max_pages = -(-vc.model_config.max_model_len // _runtime.PAGE)
            st = _runtime.make_state(cfg, self._amass_device,
                                     num_layers=len(self._amass_layers),
                                     num_blocks=int(nb), n_kv=self._amass_n_kv,
                                     G=self._amass_G, max_reqs=max_reqs,
                                     max_pages=max_pages)
            st._layer_of = ptr2layer
            self._amass_layer_k = [_split_kv(k)[0] for k in layer_kv]
            self._amass_state = st
            _notice(f"{type(st).__name__} allocated: layers={st.L} blocks={st.NB} "
                    f"reqs={max_reqs} n_kv={st.n_kv} G={st.G} max_pages={max_pages} "
                    f"rank={st.r} selector_MiB={st.bytes_per_layer() * st.L / 2**20:.1f}")
        except Exception as e:  # noqa: BLE001 - decode keeps the stock attention
            print("[amass] state allocation failed; stock attention kept:", flush=True)
            traceback.print_exception(type(e), e, e.__traceback__)
            self._amass_enabled = False
        return self._amass_state

    # ---- graph capture: dummy batches never rebuild summaries ---------------------- #
    def build_for_cudagraph_capture(self, common_attn_metadata):
        self._amass_capturing = True
        try:
            return super().build_for_cudagraph_capture(common_attn_metadata)
        finally:
            self._amass_capturing = False

    def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
        md = super().build(common_prefix_len, common_attn_metadata, fast_build)
        if self._amass_mem:
            return self._amass_tier_step(md, common_attn_metadata)
        st = self._amass_ensure_state()
        if st is None or getattr(md, "max_query_len", None) != 1:
            return md
        n_req = md.seq_lens.shape[0]
        need_derive = True
        if not self._amass_capturing:
            need_derive = self._amass_refresh(st, md, common_attn_metadata, n_req)
        if need_derive:
            from ..selection import derive_page_params
            derive_page_params(st, md.seq_lens, n_req)
        md.amass = st
        return md

    # ---- summary refresh gate -------------------------------------------------------- #
    def _amass_fns(self):
        from .. import selection as sel
        if self._amass_cfg.score in ("quad", "clse"):
            return sel.quad_build_tail, sel.quad_build_bulk, sel.quad_build_delta
        return sel.r8_build_tail, sel.r8_build_bulk, sel.r8_build_delta

    def _amass_refresh(self, st, md, cam, n_req: int) -> bool:
        """Rebuild what changed; returns whether the derive params can have changed.

        Steady batch (every row advanced by one token or is unchanged): rebuild the
        last finalised page of rows that just crossed a page boundary.  Anything else
        (first step, composition change, slot reuse): bulk the first time, then a
        tag-gated delta.  Without host seq lens, a delta every step."""
        tail, bulk, delta = self._amass_fns()
        page = _runtime.PAGE
        bt, sl = md.block_table, md.seq_lens
        host = _host_seq_lens(cam)
        if host is None:
            self._amass_prev = None
            (delta if self._amass_built_once else bulk)(st, self._amass_layer_k, bt, sl,
                                                         n_req, 0)
            self._amass_built_once = True
            return True
        cur = host[:n_req].to("cpu", torch.int64).clone()
        prev, self._amass_prev = self._amass_prev, cur
        steady = (prev is not None and prev.shape == cur.shape
                  and bool(((cur == prev + 1) | (cur == prev)).all()))
        if not steady:
            max_fin = int(cur.max().item()) // page if n_req else 0
            (delta if self._amass_built_once else bulk)(st, self._amass_layer_k, bt, sl,
                                                         n_req, max_fin)
            self._amass_built_once = True
            return True
        adv = cur == prev + 1
        crossed = adv & (cur % page == 0)
        if bool(crossed.any()):
            rows = torch.nonzero(crossed).squeeze(-1).to(bt.device)
            tail(st, self._amass_layer_k, bt, sl, n_req, rows)
        return bool((adv & (cur % page == 1)).any())


def make_builder(base: type) -> type:
    """The AMASS metadata builder class over the platform's builder class ``base``."""
    return type(f"Amass{base.__name__}", (AmassMetadataBuilderMixin, base), {})
