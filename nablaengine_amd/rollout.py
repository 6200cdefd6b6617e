"""Drivers over the step (BASELINE configs 3 and 4; reference scripts/paper_bench/ours.py:1-13 for the Jacobian,
torch_ffi.py module docstring for rollouts with torch.utils.checkpoint):

  jacobian(qpos, qvel, warm, ctrl, friction, com, *, iterations, substeps, clamp_kv, normal, clamp_soft)
      -> (J (B, 71, 99), info (B, 4)): the full step Jacobian per world, rows the outputs (qpos' in qpos form 36,
         qvel' 35), columns the inputs (qpos tangent 35, qvel 35, ctrl 29), from one taped forward and 71 one-hot
         VJPs on that tape (the reference's method), the adjoint's dispatch order computed once for the 71;
  rollout(qpos, qvel, warm, ctrls, friction, com, *, checkpoint_every=8, **step_kw) -> [(qpos_t, qvel_t)]: T steps
      under autograd, each segment of checkpoint_every steps but the last recomputed in the backward
      (torch.utils.checkpoint; their first pass writes no tapes): only the segment being differentiated and the last
      one hold tapes.

qpos tangent: a qpos-form cotangent g (36) of a state with root quaternion q maps to the tangent of
integrate_pos(q, dq) at dq = 0 (position 3, the local rotation vector 3 as 1/2 vec(q* (x) g_q), hinges 29).
"""
from . import torch_ffi

NOUT, NIN = torch_ffi.NQ + torch_ffi.NV, 2 * torch_ffi.NV + torch_ffi.NU  # 71 x 99


def qpos_tangent(qpos, g):
    """(..., B, 36) qpos-form cotangents -> (..., B, 35) tangent-form (integrate_pos's transpose at 0) at states qpos
    (B, 36)."""
    import torch
    q = qpos[:, 3:7] / qpos[:, 3:7].norm(dim=1, keepdim=True)
    gq = g[..., 3:7]
    # vec(conj(q) (x) gq): w = q0, v = -q[1:]; (w, v) (x) (s, u) = (w s - v.u, w u + s v + v x u)
    w, v = q[:, :1], -q[:, 1:]
    s, u = gq[..., :1], gq[..., 1:]
    rot = 0.5 * (w * u + s * v + torch.cross(v.expand_as(u), u, dim=-1))
    return torch.cat([g[..., :3], rot, g[..., 7:]], dim=-1)


def jacobian(qpos, qvel, warm, ctrl, friction, com, *, iterations=torch_ffi.ITERATIONS, substeps=torch_ffi.SUBSTEPS,
             clamp_kv=torch_ffi.CLAMP_KV, normal=torch_ffi.NORMAL, clamp_soft=None):
    """The step Jacobian of every world (B, 71, 99) float32 and the forward's info. The options are backward()'s
    (clamp_soft None: CLAMP_SOFT for the soft clamp), checked before anything is launched; each row is bitwise the VJP
    backward() gives for its output's one-hot cotangent."""
    import torch
    kv, nrm = torch_ffi._variant(clamp_kv, normal)
    torch_ffi._soft_delta(kv, clamp_soft)
    q1, v1, w1, info, tape = torch_ffi.forward(qpos, qvel, warm, ctrl, friction, com, iterations=iterations,
                                               substeps=substeps, tape=True)
    B = qpos.shape[0]
    eye = torch.eye(NOUT, dtype=torch.float32, device=qpos.device)  # output r's one-hot cotangent, every world
    cq = eye[:, :torch_ffi.NQ].unsqueeze(1).expand(NOUT, B, torch_ffi.NQ).contiguous()
    cv = eye[:, torch_ffi.NQ:].unsqueeze(1).expand(NOUT, B, torch_ffi.NV).contiguous()
    gq, gv, gu, _ = torch_ffi._vjp_sets(tape, friction, com, cq, cv, ctrl if kv == 2 else None, substeps=substeps,
                                        clamp_kv=kv, normal=nrm, clamp_soft=clamp_soft)
    J = torch.cat([qpos_tangent(qpos, gq), gv, gu], dim=2)  # (71, B, 99)
    return J.transpose(0, 1).contiguous(), info


def rollout(qpos, qvel, warm, ctrls, friction, com, *, checkpoint_every=8, **step_kw):
    """T = len(ctrls) differentiable steps from (qpos, qvel, warm) with the controls ctrls (T, B, 29): the states
    [(qpos_t, qvel_t)] for t = 1..T. With checkpoint_every = k > 0 each segment of k steps but the last runs once
    without writing its tapes and again in the backward, which writes them (the forward is deterministic: the
    recomputed steps are bitwise the first ones); the last segment keeps its tapes, as torch's checkpoint_sequential
    does, since the backward would recompute it first thing. k = 0 keeps every tape."""
    import torch
    from torch.utils.checkpoint import checkpoint
    T = len(ctrls)
    out = []
    q, v, w = qpos, qvel, warm

    def segment(q, v, w, *us):
        states = []
        for u in us:
            q, v, w = torch_ffi.step(q, v, w, u, friction, com, **step_kw)
            states += [q, v]
        return (w,) + tuple(states)

    def first_pass_untaped():
        """segment for checkpoint(): its first call (the forward pass, whose saved tensors the checkpoint drops) runs
        the steps without writing tapes; the recomputation in the backward writes them"""
        calls = [0]

        def run(*xs):
            calls[0] += 1
            if calls[0] == 1:
                with torch_ffi._TapeUnread():
                    return segment(*xs)
            return segment(*xs)
        return run

    k = checkpoint_every if checkpoint_every and checkpoint_every > 0 else T
    for t0 in range(0, T, k):
        us = tuple(ctrls[t] for t in range(t0, min(T, t0 + k)))
        if checkpoint_every and t0 + k < T:
            r = checkpoint(first_pass_untaped(), q, v, w, *us, use_reentrant=False)
        else:
            r = segment(q, v, w, *us)
        w = r[0]
        pairs = list(zip(r[1::2], r[2::2]))
        out += pairs
        q, v = pairs[-1]
    return out
