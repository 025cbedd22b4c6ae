"""Serving operators -- the reference's op names (serving/vllm_kernel_deltanet_op.cpp:11-58, pybind names
hybrid_recurrent_forward / fork_recurrent_state), implemented on kdn_ragged_step.

hybrid_recurrent_forward(query, key, value, beta, decay, recurrent_states, slot_mapping, output)
  query, key [num_tokens, H, d_k], value [num_tokens, H, d_v], beta, decay [num_tokens, H],
  recurrent_states [num_slots, H, d_v, D] (the reference's layout; any strides), slot_mapping [num_tokens]
  (the state slot of each token; a sequence is a run of consecutive tokens with one slot), output
  [num_tokens, H, d_v] written in place.  The reference declares this op but leaves its body empty; here
  every sequence continues from its slot with the exact delta rule (readout before update) and the
  structured lift (kernels/fwht.py:122-131), one-token sequences on the decode kernel and longer ones on
  the chunked scan, and the slots are updated in place.
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


def sequences_from_slot_mapping(slot_mapping: torch.Tensor):
    """(cu_seqlens, slots) of the runs of equal slots in slot_mapping (host tensors)."""
    sm = slot_mapping.detach().to("cpu", torch.int64)
    if sm.numel() == 0:
        return torch.zeros(1, dtype=torch.int64), torch.zeros(0, dtype=torch.int32)
    starts = torch.nonzero(torch.cat([torch.ones(1, dtype=torch.bool), sm[1:] != sm[:-1]])).flatten()
    cu = torch.cat([starts, torch.tensor([sm.numel()])]).to(torch.int64)
    slots = sm[starts].to(torch.int32)
    if torch.unique(slots).numel() != slots.numel():
        raise ValueError("hybrid_recurrent_forward: a slot appears in two separate runs of slot_mapping")
    return cu, slots


def hybrid_recurrent_forward(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, beta: torch.Tensor,
                             decay: Optional[torch.Tensor], recurrent_states: torch.Tensor,
                             slot_mapping: torch.Tensor, output: torch.Tensor,
                             cu_seqlens: Optional[torch.Tensor] = None,
                             fwht_proj: Optional[FastWalshHadamardProjection] = None,
                             normalize_input: bool = False) -> torch.Tensor:
    if recurrent_states.dim() != 4:
        raise ValueError("recurrent_states must be [num_slots, num_heads, val_dim, lifted_dim]")
    d_k, D = query.shape[-1], recurrent_states.shape[-1]
    proj = fwht_proj if fwht_proj is not None else _default_proj(d_k, D)
    if cu_seqlens is None:
        cu, slots = sequences_from_slot_mapping(slot_mapping)
    else:
        cu = torch.as_tensor(cu_seqlens, dtype=torch.int64).cpu()
        slots = slot_mapping.detach().to("cpu", torch.int64)[cu[:-1]].to(torch.int32)
    dev = query.device
    ops.ragged_step(query, key, value, beta, decay, cu, slots, recurrent_states.transpose(2, 3),
                    proj.device_omega(dev), proj.device_phase(dev), proj.tau_star_inv, normalize=normalize_input,
                    y=output)
    return output


def fork_recurrent_state(recurrent_states: torch.Tensor, parent_slot: int, child_slot: int) -> None:
    recurrent_states[child_slot].copy_(recurrent_states[parent_slot])
