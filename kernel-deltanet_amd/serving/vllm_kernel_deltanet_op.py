"""Serving operators -- the reference's op names (serving/vllm_kernel_deltanet_op.cpp:11-58, pybind names
hybrid_recurrent_forward / fork_recurrent_state), implemented on kdn_slot_step (slot map alone) and
kdn_ragged_step (host offsets).

hybrid_recurrent_forward(query, key, value, beta, decay, recurrent_states, slot_mapping, output)
  query, key [num_tokens, H, d_k], value [num_tokens, H, d_v], beta, decay [num_tokens, H],
  recurrent_states [num_slots, H, d_v, D] (the reference's layout; any strides), slot_mapping [num_tokens]
  (the state slot of each token; a sequence is a run of consecutive tokens with one slot; a negative slot
  is padding), output [num_tokens, H, d_v] written in place.  The reference declares this op but leaves
  its body empty; here every sequence continues from its slot with the exact delta rule (readout before
  update) and the structured lift (kernels/fwht.py:122-131), one-token sequences on the decode kernel and
  longer ones on the chunked scan, and the slots are updated in place.

  Two ways to describe the batch, neither of which synchronises with the host:
  - slot_mapping alone (the reference's eight arguments): kdn_slot_step finds the runs of equal slots,
    splits them into decode and prefill sequences and packs the prefills on the device, with every launch
    sized from num_tokens and the number of slots.  Distinct runs must have distinct slots (not checked);
    a slot outside recurrent_states marks padding.
  - cu_seqlens (host offsets, as a scheduler keeps them) with cu_seqlens_device (the same offsets on the
    device) and optionally seq_slots (device, one slot per sequence; default: slot_mapping at each
    sequence's first token, gathered on the device): launches sized from the actual sequence lengths.
    Device slots are not checked on the host; the kernels skip sequences whose slot is outside
    recurrent_states.
  sequences_from_slot_mapping() gives a host caller the runs and checks them (it copies slot_mapping to
  the host).
fork_recurrent_state(recurrent_states, parent_slot, child_slot)
  Copies one slot's state into another on the current stream (reference :41-58).
"""
from __future__ import annotations

from typing import Optional

import torch

from kdn import ops
from kernels.fwht import FastWalshHadamardProjection

_PROJ = {}


def _default_proj(d_k: int, D: int) -> FastWalshHadamardProjection:
    key = (d_k, D)
    if key not in _PROJ:
        _PROJ[key] = FastWalshHadamardProjection(d_k=d_k, D=D, seed=42)
    return _PROJ[key]


def sequences_from_slot_mapping(slot_mapping: torch.Tensor, num_slots: Optional[int] = None):
    """(cu_seqlens, slots) of the runs of equal slots in slot_mapping (host tensors).  Raises if a slot
    appears in two separate runs or (with num_slots) lies at or above num_slots; negative slots are
    padding runs and are kept (the step skips them)."""
    sm = slot_mapping.detach().to("cpu", torch.int64)
    if sm.numel() == 0:
        return torch.zeros(1, dtype=torch.int64), torch.zeros(0, dtype=torch.int32)
    starts = torch.nonzero(torch.cat([torch.ones(1, dtype=torch.bool), sm[1:] != sm[:-1]])).flatten()
    cu = torch.cat([starts, torch.tensor([sm.numel()])]).to(torch.int64)
    slots = sm[starts]
    live = slots[slots >= 0]
    if torch.unique(live).numel() != live.numel():
        raise ValueError("hybrid_recurrent_forward: a slot appears in two separate runs of slot_mapping")
    if num_slots is not None and live.numel() and int(live.max()) >= num_slots:
        raise ValueError(f"hybrid_recurrent_forward: slot {int(live.max())} is outside the {num_slots} state slots")
    return cu, slots.to(torch.int32)


def hybrid_recurrent_forward(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, beta: torch.Tensor,
                             decay: Optional[torch.Tensor], recurrent_states: torch.Tensor,
                             slot_mapping: torch.Tensor, output: torch.Tensor,
                             cu_seqlens=None,
                             fwht_proj: Optional[FastWalshHadamardProjection] = None,
                             normalize_input: bool = False,
                             cu_seqlens_device: Optional[torch.Tensor] = None,
                             seq_slots: Optional[torch.Tensor] = None,
                             workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    if recurrent_states.dim() != 4:
        raise ValueError("recurrent_states must be [num_slots, num_heads, val_dim, lifted_dim]")
    d_k, D = query.shape[-1], recurrent_states.shape[-1]
    proj = fwht_proj if fwht_proj is not None else _default_proj(d_k, D)
    dev = query.device
    if query.shape[0] == 0:
        return output
    if cu_seqlens is None:
        sm = slot_mapping if slot_mapping.device == dev else slot_mapping.to(dev)
        ops.slot_step(query, key, value, beta, decay, sm, recurrent_states.transpose(2, 3), proj.device_omega(dev),
                      proj.device_phase(dev), proj.tau_star_inv, normalize=normalize_input, y=output,
                      workspace=workspace)
        return output
    else:
        cu = torch.as_tensor(cu_seqlens, dtype=torch.int64)
        if cu.is_cuda:
            raise ValueError("hybrid_recurrent_forward: cu_seqlens are the host offsets; pass the device copy as "
                             "cu_seqlens_device")
        cu_dev = cu_seqlens_device
        if seq_slots is not None:
            slots = seq_slots
        elif slot_mapping.is_cuda and cu_dev is not None:
            # first token of each sequence; an empty sequence at the end would index one past the last
            # token, so indices are clamped (an empty sequence's slot is never used)
            first = cu_dev[:-1].clamp(0, slot_mapping.shape[0] - 1)
            slots = slot_mapping.index_select(0, first).to(torch.int32)
        else:
            slots = slot_mapping.detach().to("cpu", torch.int64)[cu[:-1]].to(torch.int32)
    ops.ragged_step(query, key, value, beta, decay, cu, slots, recurrent_states.transpose(2, 3),
                    proj.device_omega(dev), proj.device_phase(dev), proj.tau_star_inv, normalize=normalize_input,
                    y=output, workspace=workspace, cu_seqlens_device=cu_dev)
    return output


def fork_recurrent_state(recurrent_states: torch.Tensor, parent_slot: int, child_slot: int) -> None:
    recurrent_states[child_slot].copy_(recurrent_states[parent_slot])
