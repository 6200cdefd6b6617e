// The diagnostic counters (the reference's torch_ffi.py:56-59 DIAG order): 18 uint64 in a caller-owned device array,
// added to by k_diag_fwd / k_diag_bwd after a forward / backward, or by k_forward / k_adjoint themselves at each
// world's end when the caller passes the array to the forward or the adjoint (one launch fewer, the same counts).
//   0 fwd_calls, 1 fwd_worlds, 2 fwd_unsupported_worlds (info[3] != 0), 3 fwd_iteration_limit_worlds (the last
//   substep's iterations reached the cap), 4 tape_records, 5 refact_records, 6 nonconv_records, 7 singular_records (the
//   records' flags), 8 bwd_calls, 9 bwd_rows, 10 nonfinite_rows (a non-finite gradient), 11-13 nonfinite_{qpos,qvel,
//   ctrl}_rows, 14 nonfinite_cotangent_rows, 15 replay_mismatch_worlds, 16 fwd_contact_overflow_worlds,
//   17 fwd_row_overflow_worlds.
// The backward's info then also carries the non-finite bits (1 qpos, 2 qvel, 4 ctrl, 8 cotangent) << 16.
#pragma once

namespace g1k {
enum {
  D_FWD_CALLS = 0, D_FWD_WORLDS, D_FWD_UNSUPPORTED, D_FWD_ITER_LIMIT, D_TAPE_RECORDS, D_REFACT, D_NONCONV, D_SINGULAR,
  D_BWD_CALLS, D_BWD_ROWS, D_NONFINITE, D_NONFINITE_QPOS, D_NONFINITE_QVEL, D_NONFINITE_CTRL, D_NONFINITE_COT,
  D_REPLAY_MISMATCH, D_CONTACT_OVERFLOW, D_ROW_OVERFLOW, NDIAG
};
constexpr int NONFINITE_SHIFT = 16;
constexpr int NONFINITE_QPOS = 1, NONFINITE_QVEL = 2, NONFINITE_CTRL = 4, NONFINITE_COT = 8;
constexpr int ADJ_REPLAY_MISMATCH = 1 << 13;
constexpr int OVERFLOW_CONTACTS = 4, OVERFLOW_ROWS = 16;  // forward info[3]: contacts / rows beyond capacity dropped
}  // namespace g1k
