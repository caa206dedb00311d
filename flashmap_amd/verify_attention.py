"""Split-KV verify attention for sglang's Triton attention backend, on the gfx950 kernels.

A verify step attends L tokens per request (a draft chain or tree plus its root) to the
request's cached context and to each other. ``SplitKVVerify`` takes sglang's
``extend_attention_fwd`` arguments, as flashmap/sglang/verify_attention.py:252-474 does,
and runs ``fm_verify_attention``:

- the context is streamed once per KV head by the split-KV attention kernel, the G query
  heads sharing a KV head packed together (G * L rows per KV head, in 16-row MFMA
  blocks), the stream split evenly over the whole GPU;
- the combine kernel attends each row to its request's L verify tokens under the mask
  (causal, sglang's context + L rows, or EAGLE's QLEN_ONLY L x L blocks) and merges that
  with the context partials by their log-sum-exp.

Only shapes are read on the host, so a call can be captured in a graph. A case the
kernels do not handle returns False having done nothing (the caller then runs
extend_attention_fwd), exactly where the reference's does, plus where the gfx950
kernels need bf16 and head_dim 64 or 128.
"""

from __future__ import annotations

import torch

from . import ops

__all__ = ["SplitKVVerify"]


class SplitKVVerify:
    """extend_attention_fwd for a verify batch (flashmap/sglang/verify_attention.py:252-474).

    The kernels' workspace (packed queries, per-share partials and the plan) grows with
    the batch outside graph capture (a capture runs warm-up passes first); a replaced
    buffer is kept, as captured graphs still point at it."""

    MAX_SCRATCH_BYTES = 512 << 20
    # True when the caller's custom masks hold only the verify tokens' L x L block per
    # request (EAGLE's QLEN_ONLY layout), not a row over context + L. Set once, before
    # any graph capture. The fallback extend_attention_fwd reads only the long layout,
    # so with this set a declined masked batch is an error, not a fall-back.
    qlen_mask = False

    def __init__(self):
        self.workspace: torch.Tensor | None = None
        self._retired: list[torch.Tensor] = []

    def _scratch(self, nbytes: int, device: torch.device) -> bool:
        if self.workspace is not None and self.workspace.device == device and self.workspace.numel() >= nbytes:
            return True
        if torch.cuda.is_current_stream_capturing() or nbytes > self.MAX_SCRATCH_BYTES:
            return False
        if self.workspace is not None:
            self._retired.append(self.workspace)
        self.workspace = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        return True

    def __call__(
        self,
        q,
        k,
        v,
        o,
        k_buffer,
        v_buffer,
        qo_indptr,
        kv_indptr,
        kv_indices,
        custom_mask,
        is_causal,
        mask_indptr,
        max_len_extend,
        k_scale=1.0,
        v_scale=1.0,
        sm_scale=None,
        logit_cap=0.0,
        sliding_window_size=-1,
        sinks=None,
        window_kv_offsets=None,
        xai_temperature_len=-1,
        max_bs=None,
        **unused,
    ) -> bool:
        del window_kv_offsets, max_bs, unused
        handled = self._run(q, k, v, o, k_buffer, v_buffer, qo_indptr, kv_indptr, kv_indices, custom_mask,
                            is_causal, mask_indptr, max_len_extend, k_scale, v_scale, sm_scale, logit_cap,
                            sliding_window_size, sinks, xai_temperature_len)
        if not handled and custom_mask is not None and self.qlen_mask:
            raise RuntimeError(
                "this verify batch carries L x L masks (qlen_mask) but cannot run on the split-KV kernel, and "
                "extend_attention_fwd does not read that mask layout"
            )
        return handled

    def _run(self, q, k, v, o, k_buffer, v_buffer, qo_indptr, kv_indptr, kv_indices, custom_mask, is_causal,
             mask_indptr, max_len_extend, k_scale, v_scale, sm_scale, logit_cap, sliding_window_size, sinks,
             xai_temperature_len) -> bool:
        # The reference's declines (flashmap/sglang/verify_attention.py:382-402).
        if (logit_cap or 0) > 0 or sinks is not None or (sliding_window_size or -1) > 0:
            return False
        if (xai_temperature_len or -1) > 0 or (custom_mask is None and not is_causal):
            return False
        if not (isinstance(k_scale, (int, float)) and isinstance(v_scale, (int, float))):
            return False
        bs = qo_indptr.shape[0] - 1
        length = int(max_len_extend)
        h_q, d = q.shape[1], q.shape[2]
        h_kv, dv = k_buffer.shape[1], v_buffer.shape[-1]
        if bs < 1 or q.shape[0] != bs * length or h_q % h_kv or k_buffer.dtype != q.dtype:
            return False
        # The gfx950 kernels: bf16, head_dim 64 / 128, values as wide as keys, pool
        # and output rows readable and writable in place.
        if q.dtype != torch.bfloat16 or d not in (64, 128) or dv != d or v_buffer.dtype != q.dtype:
            return False
        if kv_indices.dtype not in (torch.int32, torch.int64):
            return False
        out = o.view(-1, h_q, dv)
        if not (ops._verify_rows(out, "o") and ops._verify_rows(k_buffer, "k_buffer")
                and ops._verify_rows(v_buffer, "v_buffer")):
            return False
        nbytes = ops.verify_workspace_bytes(bs, length, h_q, h_kv, d, 0, k_buffer.shape[0], q.device)
        if not self._scratch(nbytes, q.device):
            return False
        ops.verify_attention(
            q, k.view(-1, h_kv, d), v.view(-1, h_kv, dv), k_buffer, v_buffer, kv_indptr, kv_indices,
            custom_mask=custom_mask, mask_indptr=mask_indptr, qlen_mask=self.qlen_mask,
            sm_scale=sm_scale or d ** -0.5, k_scale=float(k_scale), v_scale=float(v_scale), out=out,
            workspace=self.workspace,
        )
        return True
