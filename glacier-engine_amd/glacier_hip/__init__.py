"""ctypes mirror of include/glacier_hip.h (the gfx950 device backend).

Loads the in-tree libglacier_hip.so and raises if it is missing: there is no
CPU fallback. Device memory for tests and benchmarks is plain torch tensors;
their addresses cross the ABI as raw pointers.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(HERE), "libglacier_hip.so")

OK = 0
SHAPE_MISMATCH = 1
DTYPE_UNSUPPORTED = 2
INVALID_ARGUMENT = 3
OUT_OF_MEMORY = 4
DEVICE_ERROR = 5
INVALID_MASK = 6
ELIGIBLE_NAN = 7
CACHE_FULL = 8
NO_DEVICE = 9
INVALID_HANDLE = 10
TRANSACTION_ACTIVE = 11
INVALID_TRANSACTION = 12
BUSY = 13
UNSUPPORTED = 14
BAD_IMAGE = 20
NOT_FOUND = 21
INVALID_CHECKPOINT = 22

F32, F16, BF16 = 0, 1, 2
ACT_Q8, ACT_F32, ACT_AUTO = 0, 1, 2


class GlacierHipError(RuntimeError):
    def __init__(self, code, what):
        super().__init__(f"{what}: status {code}")
        self.code = code


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("arch", C.c_char * 32),
                ("compute_units", C.c_uint32), ("wavefront_size", C.c_uint32),
                ("total_global_bytes", C.c_uint64), ("max_single_allocation_bytes", C.c_uint64),
                ("lds_bytes_per_block", C.c_uint32), ("l2_bytes", C.c_uint32),
                ("clock_khz", C.c_uint32), ("memory_clock_khz", C.c_uint32),
                ("memory_bus_width_bits", C.c_uint32), ("device_ordinal", C.c_uint32)]


class AllocationLimits(C.Structure):
    _fields_ = [("max_single_allocation_bytes", C.c_uint64), ("max_total_device_bytes", C.c_uint64),
                ("allocation_granularity_bytes", C.c_uint64), ("max_queue_slots", C.c_uint64)]


class Capability(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("backend_kind", C.c_uint64),
                ("device_class", C.c_uint64), ("operation_profile_bits", C.c_uint64),
                ("operator_bits", C.c_uint64), ("element_type_bits", C.c_uint64),
                ("numerical_policy_bits", C.c_uint64), ("feature_bits", C.c_uint64),
                ("max_single_allocation_bytes", C.c_uint64), ("max_total_device_bytes", C.c_uint64),
                ("max_queue_slots", C.c_uint64), ("backend_sha256", C.c_uint8 * 32),
                ("device_sha256", C.c_uint8 * 32), ("driver_sha256", C.c_uint8 * 32),
                ("placement_sha256", C.c_uint8 * 32), ("capability_sha256", C.c_uint8 * 32)]


class BufferToken(C.Structure):
    _fields_ = [("id", C.c_uint64), ("requested_bytes", C.c_uint64), ("charged_bytes", C.c_uint64)]


class BufferInfo(C.Structure):
    _fields_ = [("id", C.c_uint64), ("requested_bytes", C.c_uint64), ("charged_bytes", C.c_uint64),
                ("device_address", C.c_uint64)]


class AllocationQuote(C.Structure):
    _fields_ = [("requested_bytes", C.c_uint64), ("charged_bytes", C.c_uint64),
                ("context_epoch", C.c_uint64)]


class ArgmaxResult(C.Structure):
    _fields_ = [("token_index", C.c_uint64), ("eligible_rows", C.c_uint64),
                ("status", C.c_int32), ("reserved", C.c_int32)]


class EligibleGreedyResult(C.Structure):
    """glacier_hip_eligible_greedy_result_t (EligibleGreedyResult,
    int4_executor.zig:786-801, plus the rows this device streamed)."""
    _fields_ = [("token_index", C.c_uint64), ("eligible_rows", C.c_uint64),
                ("producer_rows", C.c_uint64), ("skipped_rows", C.c_uint64),
                ("overcomputed_rows", C.c_uint64), ("producer_runs", C.c_uint64),
                ("device_rows", C.c_uint64)]


HEAD_DOMAIN_POSTHEAD, HEAD_DOMAIN_PREHEAD = 0, 1


class ModelConfig(C.Structure):
    _fields_ = [("num_layers", C.c_uint32), ("dim", C.c_uint32), ("hidden_dim", C.c_uint32),
                ("num_heads", C.c_uint32), ("num_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("vocab_size", C.c_uint32), ("group_size", C.c_uint32),
                ("rms_eps", C.c_float), ("rope_theta", C.c_float)]


_P = C.c_void_p


class LayerHost(C.Structure):
    _fields_ = [(n, _P) for n in (
        "input_norm", "post_attn_norm", "wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down",
        "sq", "sk", "sv", "so", "s_gate", "s_up", "s_down", "bq", "bk", "bv")]


class SessionOptions(C.Structure):
    _fields_ = [("max_lanes", C.c_uint32), ("max_positions", C.c_uint32),
                ("total_pages", C.c_uint32), ("kv_dtype", C.c_int32),
                ("layer_activation", C.c_int32), ("head_activation", C.c_int32),
                ("use_graph", C.c_int32), ("prefill_chunk", C.c_int32),
                ("split_attention_o", C.c_int32)]


class PageMapRoot(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("cache_instance", C.c_uint64),
                ("generation", C.c_uint64), ("committed_len", C.c_uint64),
                ("committed_pages", C.c_uint64), ("ownership_sha256", C.c_uint8 * 32)]


class PageRef(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("abi_version", "cache_instance", "logical_page",
                                          "ownership_generation")]


class RowTxnMark(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("abi_version", "cache_id", "cache_instance", "generation",
                                          "base_len", "row_count", "root_before_generation",
                                          "root_after_generation")] + [("page_ref", PageRef)]


class ResidentLedger(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "page_count_capacity", "allocated_pages", "committed_pages", "provisional_pages",
        "reusable_pages", "page_map_bytes", "resident_tensor_payload_bytes",
        "resident_allocation_bytes", "committed_tensor_payload_bytes")]


class LaneState(C.Structure):
    _fields_ = [("kv_positions", C.c_uint64), ("published_tokens", C.c_uint64),
                ("sampling_calls", C.c_uint64), ("rng_state", C.c_uint64 * 4),
                ("output_sha256", C.c_uint8 * 32)]


CLAIM_FIELDS = ("capsule_bytes", "kv_bytes", "activation_bytes", "partial_bytes", "logits_bytes",
                "output_journal_bytes", "staging_bytes", "device_bytes", "io_bytes",
                "queue_slots")


class Claim(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in CLAIM_FIELDS]


class Limits(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("host_bytes",) + CLAIM_FIELDS]


class RequestSpec(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("tenant_key", "request_key", "request_generation",
                                          "resource_owner_key", "weight", "work_quanta",
                                          "deadline_tick")] + [("claim", Claim)]


class LaneHandle(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("scheduler_epoch", "slot_index", "slot_generation",
                                          "tenant_key", "request_key", "request_generation")]


class BankReceipt(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("bank_epoch", "slot_index", "generation", "owner_key")] + \
        [("claim", Claim), ("integrity", C.c_uint64)]


class LaneEvent(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("scheduler_epoch", C.c_uint64),
                ("event_sequence", C.c_uint64), ("kind", C.c_uint32),
                ("rejection_reason", C.c_uint32)] + \
        [(n, C.c_uint8 * 32) for n in ("previous_sha256", "event_sha256", "state_before_sha256",
                                       "state_after_sha256")] + \
        [("logical_tick_before", C.c_uint64), ("logical_tick_after", C.c_uint64)] + \
        [(n, C.c_uint32) for n in ("cursor_before", "cursor_after", "level_before",
                                   "level_after")] + \
        [("handle", LaneHandle), ("spec", RequestSpec), ("resource_receipt", BankReceipt),
         ("resource_receipt_sha256", C.c_uint8 * 32)] + \
        [(n, C.c_uint64) for n in ("remaining_before", "remaining_after", "wait_quanta",
                                   "maximum_service_gap")] + \
        [(n, C.c_uint32) for n in ("active_before", "active_after", "finished_before",
                                   "finished_after")] + \
        [("bank_used_before", Claim), ("bank_used_after", Claim)]


# ---- leased paged KV (glacier_hip_lease_* / glacier_hip_leased_kv_*) ---------
LEASE_STATUS = ["OK", "InvalidArgument", "InvalidConfiguration", "InvalidClaim", "ClaimOverflow",
                "CapacityExceeded", "ReservationSlotsExhausted", "LeaseNodesExhausted",
                "StaleReservation", "InvalidTransition", "InvalidCoordinator",
                "InvalidBindingStorage", "InvalidBinding", "InvalidLeasedPlan",
                "InvalidLeasedTransaction", "AlreadyTerminal", "TerminalRequired",
                "InvalidTerminalSeal", "ReclaimPending", "ReclaimComplete", "InvalidFreedPayload",
                "InvalidRoot", "CacheRetired", "OutOfMemory", "CacheFull", "TransactionActive",
                "InvalidTransaction", "DeviceError"]


class PublicationPermit(C.Structure):
    _fields_ = [("receipt", BankReceipt)] + \
        [(n, C.c_uint64) for n in ("request_epoch", "session_id", "sequence", "generation",
                                   "integrity")]


class LeaseTree(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("parent", BankReceipt)] + \
        [(n, C.c_uint64) for n in ("tree_key", "authority_key", "identity_generation", "generation",
                                   "structural_revision")] + \
        [("ceiling", Claim), ("current", Claim), ("active_nodes", C.c_uint32),
         ("reserved0", C.c_uint32), ("state_digest", C.c_uint64), ("integrity", C.c_uint64)]


class LeaseNode(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("parent", BankReceipt), ("tree_key", C.c_uint64),
                ("tree_identity_generation", C.c_uint64), ("node_index", C.c_uint32),
                ("reserved0", C.c_uint32), ("generation", C.c_uint64),
                ("parent_index", C.c_uint32), ("reserved1", C.c_uint32)] + \
        [(n, C.c_uint64) for n in ("parent_generation", "node_key", "tenant_key", "binding_key")] + \
        [("kind", C.c_uint32), ("reserved2", C.c_uint32), ("ceiling", Claim), ("claim", Claim),
         ("integrity", C.c_uint64)]


class LeaseBankSnapshot(C.Structure):
    _fields_ = [("used", Claim), ("peak", Claim)] + [(n, C.c_uint64) for n in (
        "peak_host_bytes", "active_reservations", "committed_receipts", "active_lease_trees",
        "active_lease_scopes", "active_lease_nodes", "reserved_unmaterialized_allocations",
        "live_allocations", "quiescing_allocations", "free_authorized_allocations",
        "successful_reservations", "successful_commits", "cancellations", "releases",
        "rejected_capacity", "rejected_slots", "lease_tree_opens", "lease_scope_opens",
        "lease_allocation_reserves", "lease_allocation_materializations", "lease_allocation_aborts",
        "lease_reclaim_prepares", "lease_reclaim_authorizations", "lease_reclaim_cancels",
        "lease_reclaim_commits", "lease_tree_closes", "rejected_lease_capacity",
        "rejected_lease_nodes")]


class PageLeaseBinding(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("state", C.c_uint32), ("has_leaf", C.c_uint32),
                ("cache_instance", C.c_uint64), ("logical_page", C.c_uint64),
                ("payload_bytes", C.c_uint64), ("scope_index", C.c_uint32),
                ("reserved0", C.c_uint32), ("scope_generation", C.c_uint64), ("leaf", LeaseNode),
                ("integrity", C.c_uint64)]


class BindingSummary(C.Structure):
    _fields_ = [("count", C.c_uint32), ("reserved0", C.c_uint32), ("payload_bytes", C.c_uint64),
                ("digest", C.c_uint8 * 32)]


class RowAllocationPlan(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "abi_version", "cache_id", "cache_instance", "base_len", "logical_page", "row_in_page",
        "root_generation", "row_txn_generation", "root_after_generation",
        "page_ownership_generation", "next_page_ownership_generation", "allocated_pages")] + \
        [("page_payload_present", C.c_uint32), ("reserved0", C.c_uint32),
         ("allocation_bytes", C.c_uint64)]


class LeasedRowPlan(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("coordinator_instance", C.c_uint64),
                ("tree", LeaseTree), ("publication_sequence", C.c_uint64),
                ("cache_plan", RowAllocationPlan), ("bindings", BindingSummary),
                ("integrity", C.c_uint64)]


class LeasedRowTxn(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("coordinator_instance", C.c_uint64),
                ("generation", C.c_uint64), ("mark", RowTxnMark),
                ("installed_new_binding", C.c_uint32), ("reserved0", C.c_uint32),
                ("bindings_digest", C.c_uint8 * 32), ("integrity", C.c_uint64)]


class TerminalSeal(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("abi_version", "coordinator_instance", "cache_id",
                                          "cache_instance")] + \
        [("scope_index", C.c_uint32), ("reserved0", C.c_uint32)] + \
        [(n, C.c_uint64) for n in ("scope_generation", "tree_identity_generation",
                                   "tree_generation", "tree_structural_revision",
                                   "tree_state_digest")] + \
        [("root", PageMapRoot), ("logical_kv_sha256", C.c_uint8 * 32),
         ("bindings", BindingSummary), ("transaction_sequence", C.c_uint64),
         ("terminal_reason", C.c_uint32), ("terminal_token", C.c_uint32),
         ("generation", C.c_uint64), ("digest", C.c_uint8 * 32)]


class FreedPayload(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("coordinator_instance", C.c_uint64),
                ("generation", C.c_uint64), ("terminal_seal_digest", C.c_uint8 * 32),
                ("permit_generation", C.c_uint64), ("root_before", PageMapRoot),
                ("root_after", PageMapRoot), ("binding_count", C.c_uint32),
                ("reserved0", C.c_uint32), ("payload_bytes", C.c_uint64),
                ("bindings_digest", C.c_uint8 * 32), ("integrity", C.c_uint64)]


class ReclaimReceipt(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("coordinator_instance", C.c_uint64),
                ("generation", C.c_uint64), ("freed", FreedPayload), ("tree_after", LeaseTree),
                ("integrity", C.c_uint64)]


_LW = [C.POINTER(LaneEvent)]

PUBLICATION_WIDTH = 4


class RootTransition(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "abi_version", "kv_row_txn_abi", "page_map_root_abi", "page_ref_abi", "cache_instance",
        "row_txn_generation", "root_before_generation", "root_after_generation",
        "root_before_len", "root_after_len", "root_before_pages", "root_after_pages")] + \
        [("root_before_ownership_sha256", C.c_uint8 * 32),
         ("root_after_ownership_sha256", C.c_uint8 * 32),
         ("logical_page", C.c_uint64), ("page_ownership_generation", C.c_uint64),
         ("installs_new_page", C.c_uint32), ("reserved", C.c_uint32),
         ("initial_logical_kv_sha256", C.c_uint8 * 32), ("row_payload_sha256", C.c_uint8 * 32),
         ("state_chain_before", C.c_uint8 * 32), ("state_chain_after", C.c_uint8 * 32)]


class LaneProposal(C.Structure):
    _fields_ = [("lane_index", C.c_uint32), ("has_kv_transition", C.c_uint32)] + \
        [(n, C.c_uint64) for n in ("step_index", "prompt_len", "kv_before", "kv_after",
                                   "kv_capacity_bytes")] + \
        [("kv_transition", RootTransition), ("output_before", C.c_uint64),
         ("output_after", C.c_uint64), ("rng_before", C.c_uint64 * 4),
         ("rng_after", C.c_uint64 * 4), ("sampling_calls_before", C.c_uint64),
         ("sampling_calls_after", C.c_uint64), ("token_id", C.c_uint32), ("terminal", C.c_uint32)]


class ServicePermit(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("abi_version", "scheduler_epoch", "coordinator_id",
                                          "coordinator_address", "permit_generation",
                                          "event_sequence")] + \
        [("handle", LaneHandle), ("logical_tick_before", C.c_uint64)] + \
        [(n, C.c_uint32) for n in ("cursor_before", "level_before", "cursor_after",
                                   "level_after")] + \
        [(n, C.c_uint64) for n in ("remaining_before", "wait_quanta", "maximum_service_gap")] + \
        [("state_before_sha256", C.c_uint8 * 32), ("chain_head_before_sha256", C.c_uint8 * 32),
         ("resource_receipt", BankReceipt), ("resource_receipt_sha256", C.c_uint8 * 32),
         ("permit_sha256", C.c_uint8 * 32)]


class WaveStage(C.Structure):
    _fields_ = [("slot", C.c_uint32), ("lane", C.c_uint32), ("stage", LaneProposal)]


WAVE_SINK = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(WaveStage), C.c_uint32)


class TokenProposal(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "abi_version", "resource_bank_abi", "resource_publication_fence_abi", "paged_kv_abi",
        "page_map_root_abi", "page_ref_abi", "page_transition_abi", "kv_row_txn_abi",
        "execution_abi", "request_epoch", "transaction_sequence", "resource_permit_generation")] + \
        [("live_mask", C.c_uint32), ("live_lane_count", C.c_uint32),
         ("kv_capacity_bytes", C.c_uint64), ("receipt", BankReceipt),
         ("lanes", LaneProposal * PUBLICATION_WIDTH)]


class PrepareAck(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("proposal_sha256", C.c_uint8 * 32),
                ("sink_epoch", C.c_uint64), ("reservation_id", C.c_uint64)]


class CommitReceipt(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("proposal_sha256", C.c_uint8 * 32),
                ("prepare_ack", PrepareAck), ("commit_sha256", C.c_uint8 * 32)]


class PublicationBinding(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("execution_abi", "request_epoch",
                                          "transaction_sequence", "resource_permit_generation",
                                          "kv_capacity_bytes")] + \
        [("receipt", BankReceipt), ("lane_index", C.c_uint32 * PUBLICATION_WIDTH),
         ("terminal", C.c_uint32 * PUBLICATION_WIDTH)]


PREPARE_ACK_ABI = 0x4750544100000001
PREPARE_ACK_V3_ABI = 0x47504C4100000003
LIFECYCLE_LIVE, LIFECYCLE_TERMINAL_RETAINED, LIFECYCLE_FREED_PENDING_UNCHARGE, \
    LIFECYCLE_RECLAIMED = 0, 1, 2, 3
TERMINAL_EOS, TERMINAL_MAX_TOKENS, TERMINAL_CANCELLED = 0, 1, 2


class AllocationSet(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("count", C.c_uint32), ("reserved", C.c_uint32),
                ("payload_bytes", C.c_uint64), ("sha256", C.c_uint8 * 32)]


class LeaseTreeCommitment(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("abi_version", "tree_key", "identity_generation",
                                          "generation", "structural_revision")] + \
        [("ceiling", Claim), ("current", Claim), ("active_nodes", C.c_uint32),
         ("reserved", C.c_uint32), ("state_digest", C.c_uint64), ("token_integrity", C.c_uint64)]


class ResourceCommitment(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("lane_index", C.c_uint32), ("lifecycle", C.c_uint32),
                ("coordinator_instance", C.c_uint64), ("cache_instance", C.c_uint64),
                ("scope_index", C.c_uint32), ("reserved0", C.c_uint32),
                ("scope_generation", C.c_uint64), ("root", PageMapRoot),
                ("kv_state_chain_after", C.c_uint8 * 32), ("has_canonical_after", C.c_uint32),
                ("reserved1", C.c_uint32), ("canonical_after_sha256", C.c_uint8 * 32),
                ("has_terminal_generation", C.c_uint32), ("reserved2", C.c_uint32),
                ("terminal_generation", C.c_uint64), ("has_binding_summary", C.c_uint32),
                ("reserved3", C.c_uint32), ("binding_summary", BindingSummary),
                ("allocation_set", AllocationSet)]


class LaneProposalV3(C.Structure):
    _fields_ = [("lane_index", C.c_uint32), ("has_kv_transition", C.c_uint32)] + \
        [(n, C.c_uint64) for n in ("step_index", "prompt_len", "kv_before", "kv_after")] + \
        [("kv_transition", RootTransition), ("output_before", C.c_uint64),
         ("output_after", C.c_uint64), ("output_sha256", C.c_uint8 * 32),
         ("rng_before", C.c_uint64 * 4), ("rng_after", C.c_uint64 * 4),
         ("sampling_calls_before", C.c_uint64), ("sampling_calls_after", C.c_uint64),
         ("token_id", C.c_uint32), ("terminal_reason", C.c_uint32)]


class TokenProposalV3(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "abi_version", "resource_bank_abi", "resource_lease_tree_abi",
        "resource_publication_fence_abi", "leased_paged_kv_abi", "paged_kv_abi",
        "page_transition_abi", "execution_abi", "request_epoch", "transaction_sequence",
        "resource_permit_generation")] + \
        [("live_mask", C.c_uint32), ("live_lane_count", C.c_uint32),
         ("parent_receipt", BankReceipt), ("tree", LeaseTreeCommitment),
         ("resources", ResourceCommitment * PUBLICATION_WIDTH),
         ("lanes", LaneProposalV3 * PUBLICATION_WIDTH)]


class CommandToken(C.Structure):
    _fields_ = [("context_nonce", C.c_uint64 * 4), ("generation", C.c_uint64)]


class AsyncSubmission(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("token", CommandToken),
                ("submission_binding", C.c_uint8 * 32), ("disposition", C.c_uint32),
                ("reserved", C.c_uint32)]


class AsyncCompletion(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("token", CommandToken),
                ("submission_binding", C.c_uint8 * 32), ("current_allocated_before", C.c_uint64),
                ("current_allocated_after", C.c_uint64), ("gpu_start_time", C.c_double),
                ("gpu_end_time", C.c_double), ("error_code", C.c_int64)] + \
        [(n, C.c_uint32) for n in ("state", "command_status", "error_domain_kind",
                                   "error_present", "callback_fault", "reserved")]


class GlrtOpenOptions(C.Structure):
    _fields_ = [("verify_payload_crc", C.c_int32), ("verify_payload_digest", C.c_int32),
                ("allow_v1", C.c_int32), ("check_source_fingerprint", C.c_int32),
                ("expected_source_fingerprint", C.c_uint8 * 32)]


class GlrtInfo(C.Structure):
    _fields_ = [("error", C.c_uint32), ("version", C.c_uint32), ("record_count", C.c_uint64),
                ("data_offset", C.c_uint64), ("file_size", C.c_uint64),
                ("source_fingerprint", C.c_uint8 * 32), ("abi_fingerprint", C.c_uint8 * 32)] + \
        [(n, C.c_uint32) for n in ("dim", "hidden_dim", "layers", "vocab", "heads", "head_dim",
                                   "kv_heads", "tie_embeddings")] + \
        [("rms_eps", C.c_float), ("rope_theta", C.c_float)]


class GlrtRecord(C.Structure):
    _fields_ = [("layer_idx", C.c_uint32), ("kind", C.c_uint32), ("role", C.c_uint16),
                ("encoding", C.c_uint16), ("packed_layout", C.c_uint16),
                ("pair_nibble_layout", C.c_uint16)] + \
        [(n, C.c_uint32) for n in ("group_size", "out_f", "in_f", "flags", "payload_crc32",
                                   "reserved")] + \
        [("num_elements", C.c_uint64), ("offset", C.c_uint64 * 5), ("length", C.c_uint64 * 5),
         ("payload_digest", C.c_uint8 * 32)]


class GlrtLoadReport(C.Structure):
    _fields_ = [("error", C.c_uint32), ("separate_mlp", C.c_uint32), ("int4_records", C.c_uint64),
                ("raw_records", C.c_uint64), ("inexact_scales", C.c_uint64),
                ("uploaded_bytes", C.c_uint64)]


class GlacierHeader(C.Structure):
    _fields_ = [("version", C.c_uint32), ("header_size", C.c_uint32)] + \
        [(n, C.c_uint64) for n in ("meta_offset", "meta_len", "num_pages", "page_index_offset",
                                   "page_data_offset")] + \
        [("page_size_log2", C.c_uint32), ("reserved", C.c_uint32),
         ("container_bytes", C.c_uint64)]


class GlacierPage(C.Structure):
    _fields_ = [("page_id", C.c_uint64), ("layer_idx", C.c_uint32), ("tensor_kind", C.c_uint32),
                ("row_start", C.c_uint64), ("row_end", C.c_uint64), ("precision", C.c_uint32),
                ("quant_group", C.c_uint32), ("data_offset", C.c_uint64),
                ("data_len", C.c_uint64), ("crc32", C.c_uint32), ("reserved", C.c_uint32)]


class GlacierAssembly(C.Structure):
    _fields_ = [("error", C.c_uint32), ("num_layers", C.c_uint32)] + \
        [(n, C.c_uint64) for n in ("dim", "hidden_dim", "vocab_size", "groups", "int4_groups")] + \
        [("sha256", C.c_uint8 * 32)]


class GlacierLoadReport(C.Structure):
    _fields_ = [("error", C.c_uint32), ("int4_tensors", C.c_uint32), ("raw_tensors", C.c_uint32),
                ("reserved", C.c_uint32), ("inexact_scales", C.c_uint64),
                ("uploaded_bytes", C.c_uint64), ("config", ModelConfig)]


GLACIER_ERRORS = [
    "Ok", "TruncatedHeader", "BadMagic", "BadVersion", "BadHeaderSize", "BadPageSize",
    "BadReservedField", "BadLayout", "MetadataTooLarge", "IndexTooLarge", "LayoutOverflow",
    "TruncatedMeta", "TruncatedIndex", "BadMetadata", "BadTensorKind", "BadPrecision",
    "BadPageId", "BadRowRange", "EmptyPage", "BadQuantGroup", "PageGeometryTooLarge",
    "BadPageGeometry", "UnsupportedPrecision", "NonContiguousPayload", "TruncatedPage",
    "TrailingBytes", "CrcMismatch", "BadQuantPayload", "BufferTooSmall", "EmptyStreamBuffer",
    "FileError", "SizeMismatch", "BadGroupSize", "TruncatedScales", "TruncatedPacked",
    "InvalidPayloadSize", "InvalidValue", "NoLayers", "MissingTensor", "BadPayload",
    "Unsupported", "InvalidArgument"]


class PageImageInfo(C.Structure):
    _fields_ = [("error", C.c_uint32), ("reserved", C.c_uint32), ("source_root", PageMapRoot),
                ("num_layers", C.c_uint64), ("dim", C.c_uint64), ("max_seq", C.c_uint64),
                ("source_ref", PageRef), ("committed_rows", C.c_uint64),
                ("payload_element_count", C.c_uint64), ("payload_offset", C.c_uint64),
                ("challenge_sha256", C.c_uint8 * 32), ("image_sha256", C.c_uint8 * 32)]


class CheckpointRestore(C.Structure):
    _fields_ = [("abi_version", C.c_uint64), ("source_root", PageMapRoot),
                ("target_root", PageMapRoot), ("restored_pages", C.c_uint64),
                ("restored_payload_bytes", C.c_uint64), ("error", C.c_uint32),
                ("reserved", C.c_uint32)]


# glacier_hip_page_image_error, by the reference's error names
PAGE_IMAGE_ERRORS = ["Ok", "InvalidLength", "InvalidMagic", "InvalidAbi", "InvalidFlags",
                     "InvalidPageImage", "CapacityExceeded", "UnsafeDestination",
                     "ForeignCheckpoint", "InvalidCheckpoint", "InvalidRestorePlan",
                     "ArithmeticOverflow"]


# glacier_hip_glrt_error, by the reference's error names
GLRT_ERRORS = ["Ok", "TruncatedHeader", "BadMagic", "BadVersion", "BadHeaderSize", "BadRecordSize",
               "BadAlignment", "BadConfig", "BadReservedField", "HeaderCrcMismatch",
               "LegacyVersionDisabled", "BadHeader", "BadBounds", "SourceFingerprintMismatch",
               "AbiFingerprintMismatch", "IndexCrcMismatch", "TruncatedIndex", "BadTensorKind",
               "BadEncoding", "BadPackedLayout", "BadRole", "BadPairNibbleLayout", "BadFlags",
               "BadVersionedRecord", "MissingDigest", "BadTensorShape", "MissingScales",
               "OverlappingPayload", "DuplicateRecord", "CrcMismatch", "DigestMismatch",
               "FileError", "MissingTensor", "BadPayload", "NoLayers", "Unsupported"]


COMMAND_PENDING, COMMAND_COMPLETED, COMMAND_ERROR, COMMAND_UNKNOWN = 1, 2, 3, 4

# (name, restype, argtypes) for every exported symbol of include/glacier_hip.h
_SIGS = [
    ("glacier_hip_abi_version", C.c_uint64, []),
    ("glacier_hip_init", _P, [C.c_int]),
    ("glacier_hip_deinit", C.c_int, [_P]),
    ("glacier_hip_device_info", C.c_int, [_P, C.POINTER(DeviceInfo)]),
    ("glacier_hip_allocation_limits", C.c_int, [_P, C.POINTER(AllocationLimits)]),
    ("glacier_hip_last_error", C.c_char_p, [_P]),
    ("glacier_hip_synchronize", C.c_int, [_P]),
    ("glacier_hip_device_capability_v1", C.c_int, [_P, C.POINTER(Capability)]),
    ("glacier_hip_buffer_create", C.c_int, [_P, C.c_uint64, C.POINTER(BufferToken)]),
    ("glacier_hip_buffer_info", C.c_int, [_P, C.POINTER(BufferToken), C.POINTER(BufferInfo)]),
    ("glacier_hip_buffer_release", C.c_int, [_P, C.POINTER(BufferToken)]),
    ("glacier_hip_live_buffer_count", C.c_int, [_P, C.POINTER(C.c_uint64)]),
    ("glacier_hip_allocation_quote", C.c_int, [_P, C.c_uint64, C.POINTER(AllocationQuote)]),
    ("glacier_hip_allocation_allocate", C.c_int,
     [_P, C.POINTER(AllocationQuote), C.POINTER(BufferToken)]),
    ("glacier_hip_allocation_free", C.c_int, [_P, C.POINTER(BufferToken)]),
    ("glacier_hip_live_device_bytes", C.c_int, [_P, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    ("glacier_hip_int4_weight_create", _P,
     [_P, _P, C.c_uint64, _P, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32]),
    ("glacier_hip_int4_weight_create_f16scales", _P,
     [_P, _P, C.c_uint64, _P, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32]),
    ("glacier_hip_int4_weight_destroy", None, [_P]),
    ("glacier_hip_live_weight_count", C.c_int, [_P, C.POINTER(C.c_uint64)]),
    ("glacier_hip_int4_weight_device_bytes", C.c_uint64, [_P]),
    ("glacier_hip_int4_matvec_dispatch", C.c_int, [_P, _P, _P, C.c_uint64, _P, C.c_uint64]),
    ("glacier_hip_int4_registered_buffers_submit_async", C.c_int,
     [_P] + [C.POINTER(BufferToken)] * 4 + [_P, C.c_uint64, _P, C.c_uint64, _P, C.c_uint64,
                                            C.c_uint32, C.c_uint32, C.c_uint32, _P,
                                            C.POINTER(AsyncSubmission)]),
    ("glacier_hip_registered_dispatch_poll", C.c_int,
     [_P, C.POINTER(CommandToken), _P, C.POINTER(AsyncCompletion)]),
    ("glacier_hip_registered_dispatch_wait", C.c_int,
     [_P, C.POINTER(CommandToken), _P, C.POINTER(AsyncCompletion)]),
    ("glacier_hip_registered_dispatch_finalize", C.c_int,
     [_P, C.POINTER(CommandToken), _P, C.POINTER(AsyncCompletion)]),
    ("glacier_hip_int4_registered_output_read", C.c_int,
     [_P, C.POINTER(CommandToken), _P, C.POINTER(AsyncCompletion), C.POINTER(BufferToken), _P,
      C.c_uint64]),
    ("glacier_hip_live_command_count", C.c_int, [_P, C.POINTER(C.c_uint64)]),
    ("glacier_hip_int4_gemv", C.c_int, [_P, _P, _P, C.c_int, C.c_uint32, _P, _P, C.c_int, _P]),
    ("glacier_hip_int4_gemv_noalloc", C.c_int,
     [_P, _P, _P, C.c_int, C.c_uint32, _P, _P, C.c_int, _P]),
    ("glacier_hip_activation_bytes", C.c_uint64, [C.c_uint32, C.c_uint32, C.c_int]),
    ("glacier_hip_activation_prepare", C.c_int,
     [_P, _P, C.c_int, C.c_uint32, C.c_uint32, C.c_int, _P, _P]),
    ("glacier_hip_int4_gemv_prepared", C.c_int, [_P, _P, _P, C.c_uint32, C.c_int, _P, _P, _P]),
    ("glacier_hip_rmsnorm", C.c_int, [_P, _P, _P, C.c_uint32, C.c_uint32, C.c_float, _P, _P]),
    ("glacier_hip_paged_attention", C.c_int,
     [_P, _P, _P, C.c_int, _P, C.c_uint32, _P, C.c_uint32, C.c_uint32, C.c_uint32,
      C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _P, _P]),
    ("glacier_hip_paged_attention_o", C.c_int,
     [_P, _P, _P, _P, C.c_uint32, _P, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
      C.c_uint32, C.c_uint32, _P, _P, _P]),
    ("glacier_hip_paged_attention_prefill", C.c_int,
     [_P, _P, _P, _P, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
      C.c_uint32, C.c_uint32, _P, _P]),
    ("glacier_hip_argmax", C.c_int, [_P, _P, C.c_uint64, C.c_uint32, _P, _P]),
    ("glacier_hip_eligible_argmax", C.c_int,
     [_P, _P, C.c_uint64, _P, C.c_uint64, C.c_uint32, C.POINTER(ArgmaxResult), _P]),
    ("glacier_hip_int4_eligible_greedy", C.c_int,
     [_P, _P, _P, C.c_uint32, _P, C.c_uint64, C.c_int, C.POINTER(EligibleGreedyResult), _P]),
    ("glacier_hip_model_create", _P, [_P, C.POINTER(ModelConfig)]),
    ("glacier_hip_model_set_layer", C.c_int, [_P, C.c_uint32, C.POINTER(LayerHost)]),
    ("glacier_hip_model_set_globals", C.c_int, [_P, _P, _P, _P, _P]),
    ("glacier_hip_model_init_random", C.c_int, [_P, C.c_uint64]),
    ("glacier_hip_model_destroy", None, [_P]),
    ("glacier_hip_model_weight_bytes", C.c_uint64, [_P]),
    ("glacier_hip_model_quote", C.c_int,
     [_P, C.POINTER(ModelConfig), C.c_int, C.POINTER(AllocationQuote)]),
    ("glacier_hip_session_quote", C.c_int,
     [_P, C.POINTER(SessionOptions), C.POINTER(AllocationQuote)]),
    ("glacier_hip_session_create", _P, [_P, C.POINTER(SessionOptions)]),
    ("glacier_hip_session_destroy", None, [_P]),
    ("glacier_hip_session_lane_begin", C.c_int, [_P, C.c_uint32, C.c_uint64]),
    ("glacier_hip_session_prefill", C.c_int, [_P, C.c_uint32, _P, C.c_uint32, _P, _P]),
    ("glacier_hip_session_decode_step", C.c_int, [_P, _P, _P, C.c_uint32, _P, _P, _P]),
    ("glacier_hip_session_lane_root", C.c_int, [_P, C.c_uint32, C.POINTER(PageMapRoot)]),
    ("glacier_hip_session_lane_state", C.c_int, [_P, C.c_uint32, C.POINTER(LaneState)]),
    ("glacier_hip_session_lane_kv_sha256", C.c_int, [_P, C.c_uint32, _P]),
    ("glacier_hip_session_read_kv_row", C.c_int,
     [_P, C.c_uint32, C.c_uint32, C.c_int, C.c_uint32, _P]),
    ("glacier_hip_session_page_of", C.c_int, [_P, C.c_uint32, C.c_uint32, C.POINTER(C.c_int32)]),
    ("glacier_hip_session_page_generation", C.c_int,
     [_P, C.c_uint32, C.c_uint32, C.POINTER(C.c_uint64)]),
    ("glacier_hip_session_set_head_domain", C.c_int, [_P, C.c_int]),
    ("glacier_hip_kv_pages_create", _P, [C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]),
    ("glacier_hip_kv_pages_destroy", None, [_P]),
    ("glacier_hip_kv_pages_begin_row", C.c_int, [_P, C.POINTER(RowTxnMark)]),
    ("glacier_hip_kv_pages_commit_row", C.c_int, [_P, C.POINTER(RowTxnMark)]),
    ("glacier_hip_kv_pages_abort_row", C.c_int, [_P, C.POINTER(RowTxnMark)]),
    ("glacier_hip_kv_pages_staged_root", C.c_int,
     [_P, C.POINTER(RowTxnMark), C.POINTER(PageMapRoot), C.POINTER(PageMapRoot)]),
    ("glacier_hip_kv_pages_reset", C.c_int, [_P]),
    ("glacier_hip_kv_pages_root", C.c_int, [_P, C.POINTER(PageMapRoot)]),
    ("glacier_hip_kv_pages_page", C.c_int,
     [_P, C.c_uint32, C.POINTER(C.c_int32), C.POINTER(C.c_uint64)]),
    ("glacier_hip_kv_pages_validate_page_ref", C.c_int, [_P, C.POINTER(PageRef)]),
    ("glacier_hip_kv_pages_ledger", C.c_int, [_P, C.POINTER(ResidentLedger)]),
    ("glacier_hip_session_inject_failure", C.c_int, [_P, C.c_int]),
    ("glacier_hip_session_trace_layers", C.c_int, [_P, C.c_int]),
    ("glacier_hip_session_probe_kernel", C.c_int, [_P, C.c_int]),
    ("glacier_hip_session_probe_replay", C.c_int, [_P, C.c_int, C.c_uint32, C.POINTER(C.c_double)]),
    ("glacier_hip_session_probe_read", C.c_int, [_P, C.POINTER(C.c_double), C.POINTER(C.c_uint64)]),
    ("glacier_hip_session_layer_trace", C.c_int, [_P, _P, C.POINTER(C.c_uint32)]),
    ("glacier_hip_session_prefill_staged", C.c_int, [_P, C.c_uint32, _P, C.c_uint32, _P, _P]),
    ("glacier_hip_session_step_prepare", C.c_int,
     [_P, _P, _P, C.c_uint32, _P, C.POINTER(PublicationBinding), C.POINTER(TokenProposal), _P,
      _P, _P]),
    ("glacier_hip_session_step_commit", C.c_int,
     [_P, C.POINTER(PrepareAck), C.POINTER(CommitReceipt)]),
    ("glacier_hip_session_step_abort", C.c_int, [_P]),
    ("glacier_hip_token_proposal_sha256", C.c_int, [C.POINTER(TokenProposal), _P]),
    ("glacier_hip_token_commit_sha256", C.c_int, [_P, C.POINTER(PrepareAck), _P]),
    ("glacier_hip_token_sequence_sha256", C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p]),
    ("glacier_hip_token_proposal_v3_sha256", C.c_int, [C.POINTER(TokenProposalV3), _P]),
    ("glacier_hip_token_commit_v3_sha256", C.c_int, [_P, C.POINTER(PrepareAck), _P]),
    ("glacier_hip_session_step_prepare_v3", C.c_int,
     [_P, _P, _P, C.c_uint32, _P, C.POINTER(PublicationBinding), _P, C.POINTER(TokenProposalV3),
      _P, _P]),
    ("glacier_hip_synth_int4", None, [C.c_uint64, C.c_uint64, _P, C.c_uint64]),
    ("glacier_hip_synth_scales_f16", None, [C.c_uint64, C.c_uint64, C.c_float, _P, C.c_uint64]),
    ("glacier_hip_synth_normal_f32", None, [C.c_uint64, C.c_uint64, C.c_float, _P, C.c_uint64]),
    ("glacier_hip_synth_tokens", None, [C.c_uint64, C.c_uint64, C.c_uint32, _P, C.c_uint64]),
    ("glacier_hip_synth_tensor_id", C.c_uint64, [C.c_uint32, C.c_uint32]),
    ("glacier_hip_f16_to_f32", C.c_float, [C.c_uint16]),
    ("glacier_hip_lane_weave_create", _P,
     [C.c_uint32, C.POINTER(Limits), C.c_uint64, C.c_uint64, _P, C.c_uint32, C.c_uint64,
      C.c_uint64]),
    ("glacier_hip_lane_weave_destroy", None, [_P]),
    ("glacier_hip_lane_weave_admit", C.c_int,
     [_P, C.POINTER(RequestSpec), C.POINTER(C.c_int), C.POINTER(LaneHandle)] + _LW),
    ("glacier_hip_lane_weave_serve_one", C.c_int, [_P] + _LW),
    ("glacier_hip_lane_weave_plan_wave", C.c_int, [_P, C.c_uint32, _P, C.POINTER(C.c_uint32)]),
    ("glacier_hip_lane_weave_retire", C.c_int, [_P, C.POINTER(LaneHandle)] + _LW),
    ("glacier_hip_lane_weave_cancel", C.c_int, [_P, C.POINTER(LaneHandle)] + _LW),
    ("glacier_hip_lane_weave_close", C.c_int, [_P] + _LW),
    ("glacier_hip_lane_weave_slot", C.c_int,
     [_P, C.c_uint32, C.POINTER(LaneHandle), C.POINTER(C.c_uint32), C.POINTER(C.c_uint64)]),
    ("glacier_hip_lane_weave_chain_head", C.c_int, [_P, _P]),
    ("glacier_hip_lane_weave_state_sha256", C.c_int, [_P, _P]),
    ("glacier_hip_session_lane_weave_wave", C.c_int,
     [_P, _P, _P, C.c_uint32, _P, _P, C.c_uint32, _P, _P, C.POINTER(C.c_uint32)]),
    ("glacier_hip_session_lane_weave_wave_staged", C.c_int,
     [_P, _P, _P, C.c_uint32, _P, _P, C.c_uint32, WAVE_SINK, _P, _P, _P, C.POINTER(C.c_uint32)]),
    ("glacier_hip_lane_weave_prepare_service", C.c_int, [_P, C.POINTER(ServicePermit)]),
    ("glacier_hip_lane_weave_commit_service", C.c_int,
     [_P, C.POINTER(ServicePermit), C.POINTER(LaneEvent)]),
    ("glacier_hip_lane_weave_abort_service", C.c_int, [_P, C.POINTER(ServicePermit)]),
    ("glacier_hip_service_permit_sha256", C.c_int, [C.POINTER(ServicePermit), _P]),
    ("glacier_hip_page_image_bytes", C.c_uint64, [C.c_uint64, C.c_uint64, C.c_uint64]),
    ("glacier_hip_page_image_encode_canonical", C.c_int,
     [C.POINTER(PageMapRoot), C.c_uint64, C.c_uint64, C.c_uint64, C.POINTER(PageRef), C.c_uint64,
      _P, C.c_uint64, _P, _P, C.c_uint64, C.POINTER(C.c_uint64), C.POINTER(PageImageInfo)]),
    ("glacier_hip_page_image_decode", C.c_int, [_P, C.c_uint64, _P, C.POINTER(PageImageInfo)]),
    ("glacier_hip_session_encode_page_image", C.c_int,
     [_P, C.c_uint32, C.c_uint32, _P, _P, C.c_uint64, C.POINTER(C.c_uint64),
      C.POINTER(PageImageInfo)]),
    ("glacier_hip_session_restore_checkpoint", C.c_int,
     [_P, C.c_uint32, C.POINTER(C.c_char_p), C.POINTER(C.c_uint64), C.c_uint32, _P, C.c_uint64,
      C.POINTER(CheckpointRestore), C.POINTER(PageRef)]),
    ("glacier_hip_glrt_open", C.c_int,
     [C.c_char_p, C.POINTER(GlrtOpenOptions), C.POINTER(_P), C.POINTER(GlrtInfo)]),
    ("glacier_hip_glrt_close", None, [_P]),
    ("glacier_hip_glrt_record_at", C.c_int, [_P, C.c_uint64, C.POINTER(GlrtRecord)]),
    ("glacier_hip_glrt_find", C.c_int, [_P, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(GlrtRecord)]),
    ("glacier_hip_glrt_stream", C.c_int,
     [_P, C.POINTER(GlrtRecord), C.c_uint32, C.POINTER(_P), C.POINTER(C.c_uint64)]),
    ("glacier_hip_glrt_identity", C.c_int, [_P, _P, C.POINTER(C.c_uint64)]),
    ("glacier_hip_model_load_glrt", _P, [_P, _P, C.POINTER(GlrtLoadReport)]),
    ("glacier_hip_glacier_error_name", C.c_char_p, [C.c_uint32]),
    ("glacier_hip_glacier_open", C.c_int, [C.c_char_p, C.POINTER(_P)]),
    ("glacier_hip_glacier_close", None, [_P]),
    ("glacier_hip_glacier_header", C.c_int, [_P, C.POINTER(GlacierHeader)]),
    ("glacier_hip_glacier_page", C.c_int, [_P, C.c_uint64, C.POINTER(GlacierPage)]),
    ("glacier_hip_glacier_metadata", C.c_int, [_P, C.POINTER(_P), C.POINTER(C.c_uint64)]),
    ("glacier_hip_glacier_read_page", C.c_int, [_P, C.c_uint64, _P, C.c_uint64]),
    ("glacier_hip_glacier_read_page_f32", C.c_int,
     [_P, C.c_uint64, _P, C.c_uint64, C.POINTER(C.c_uint64)]),
    ("glacier_hip_glacier_validate_crcs", C.c_int, [_P, C.c_uint64]),
    ("glacier_hip_glacier_identity", C.c_int, [_P, _P, C.POINTER(C.c_uint64)]),
    ("glacier_hip_glacier_source_fingerprint", C.c_int, [_P, _P]),
    ("glacier_hip_glacier_assemble", C.c_int, [_P, C.POINTER(GlacierAssembly)]),
    ("glacier_hip_qio_encode_f32", C.c_int,
     [_P, C.c_uint64, C.c_uint32, C.c_uint32, _P, C.c_uint64, C.POINTER(C.c_uint64)]),
    ("glacier_hip_qio_decode_f32", C.c_int,
     [_P, C.c_uint64, _P, C.c_uint64, C.POINTER(C.c_uint64)]),
    ("glacier_hip_model_load_glacier", _P,
     [_P, _P, C.POINTER(ModelConfig), C.c_int, C.POINTER(GlacierLoadReport)]),
    ("glacier_hip_lease_bank_create", _P, [C.c_uint32, C.c_uint32, C.POINTER(Limits), C.c_uint64]),
    ("glacier_hip_lease_bank_destroy", None, [_P]),
    ("glacier_hip_lease_bank_reserve", C.c_int,
     [_P, C.c_uint64, C.POINTER(Claim), C.POINTER(BankReceipt)]),
    ("glacier_hip_lease_bank_commit", C.c_int, [_P, C.POINTER(BankReceipt), C.POINTER(BankReceipt)]),
    ("glacier_hip_lease_bank_cancel", C.c_int, [_P, C.POINTER(BankReceipt)]),
    ("glacier_hip_lease_bank_release", C.c_int, [_P, C.POINTER(BankReceipt)]),
    ("glacier_hip_lease_tree_open", C.c_int,
     [_P, C.POINTER(BankReceipt), C.c_uint64, C.c_uint64, C.POINTER(Claim), C.POINTER(LeaseTree)]),
    ("glacier_hip_lease_scope_open", C.c_int,
     [_P, C.POINTER(LeaseTree), C.c_uint64, C.c_uint64, C.POINTER(Claim), C.POINTER(LeaseNode)]),
    ("glacier_hip_lease_tree_close", C.c_int, [_P, C.POINTER(LeaseTree)]),
    ("glacier_hip_lease_tree_validate", C.c_int, [_P, C.POINTER(LeaseTree)]),
    ("glacier_hip_lease_node_validate", C.c_int, [_P, C.POINTER(LeaseTree), C.POINTER(LeaseNode)]),
    ("glacier_hip_lease_session_bind", C.c_int, [_P, C.POINTER(LeaseTree), C.c_uint64, C.c_uint64]),
    ("glacier_hip_lease_session_close", C.c_int,
     [_P, C.POINTER(BankReceipt), C.c_uint64, C.c_uint64, C.c_uint64]),
    ("glacier_hip_lease_bank_snapshot", C.c_int, [_P, C.POINTER(LeaseBankSnapshot)]),
    ("glacier_hip_lease_publication_begin", C.c_int,
     [_P, C.POINTER(LeaseTree), C.c_uint64, C.c_uint64, C.c_uint64,
      C.POINTER(PublicationPermit)]),
    ("glacier_hip_lease_publication_commit", C.c_int, [_P, C.POINTER(PublicationPermit)]),
    ("glacier_hip_lease_publication_abort", C.c_int, [_P, C.POINTER(PublicationPermit)]),
    ("glacier_hip_leased_kv_create", C.c_int,
     [_P, C.POINTER(LeaseTree), C.POINTER(LeaseNode), _P, C.POINTER(PageLeaseBinding), C.c_uint32,
      C.c_uint64, C.c_uint64, C.POINTER(C.c_uint64), C.POINTER(_P)]),
    ("glacier_hip_leased_kv_create_for_lane", C.c_int,
     [_P, C.POINTER(LeaseTree), C.POINTER(LeaseNode), _P, C.c_uint32, C.POINTER(PageLeaseBinding),
      C.c_uint32, C.c_uint64, C.c_uint64, C.POINTER(C.c_uint64), C.POINTER(_P)]),
    ("glacier_hip_leased_kv_destroy", None, [_P]),
    ("glacier_hip_leased_kv_plan_next_row", C.c_int, [_P, C.POINTER(LeasedRowPlan)]),
    ("glacier_hip_leased_kv_begin_row", C.c_int,
     [_P, C.POINTER(LeasedRowPlan), C.POINTER(LeasedRowTxn)]),
    ("glacier_hip_leased_kv_commit_row", C.c_int,
     [_P, C.POINTER(LeasedRowTxn), C.POINTER(PageMapRoot)]),
    ("glacier_hip_leased_kv_abort_row", C.c_int, [_P, C.POINTER(LeasedRowTxn)]),
    ("glacier_hip_leased_kv_binding_summary", C.c_int, [_P, C.POINTER(BindingSummary)]),
    ("glacier_hip_leased_kv_lifecycle", C.c_int, [_P, C.POINTER(C.c_uint32)]),
    ("glacier_hip_leased_kv_allocation_set", C.c_int, [_P, C.POINTER(AllocationSet)]),
    ("glacier_hip_leased_kv_root", C.c_int, [_P, C.POINTER(PageMapRoot)]),
    ("glacier_hip_leased_kv_kv_sha256", C.c_int, [_P, _P]),
    ("glacier_hip_leased_kv_seal_terminal", C.c_int,
     [_P, C.POINTER(PageMapRoot), _P, C.c_uint64, C.c_uint32, C.c_uint32,
      C.POINTER(TerminalSeal)]),
    ("glacier_hip_leased_kv_begin_reclaim", C.c_int,
     [_P, C.POINTER(TerminalSeal), C.c_uint64, C.POINTER(FreedPayload)]),
    ("glacier_hip_leased_kv_commit_reclaim", C.c_int,
     [_P, C.POINTER(FreedPayload), C.POINTER(ReclaimReceipt)]),
    ("glacier_hip_leased_kv_reclaim_for_teardown", C.c_int, [_P, C.c_uint64]),
    ("glacier_hip_leased_kv_terminal_seal", C.c_int, [_P, C.POINTER(TerminalSeal), _P, _P]),
    ("glacier_hip_kv_pages_append_row", C.c_int,
     [_P, C.POINTER(RowTxnMark), C.c_uint32, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
    ("glacier_hip_kv_pages_kv_sha256", C.c_int, [_P, _P]),
    ("glacier_hip_kv_pages_is_retired", C.c_int, [_P, C.POINTER(C.c_int32)]),
    ("glacier_hip_kv_pages_set_pool_capacity", C.c_int, [_P, C.c_uint32]),
]

_lib = None


def lib():
    """Load libglacier_hip.so; raise when it has not been built."""
    global _lib
    if _lib is None:
        # One HIP runtime per process: torch ships its own libamdhip64 (soname
        # libamdhip64.so.7). Loading torch first lets this library bind to that
        # same runtime by soname; loading /opt/rocm's copy first would leave two
        # runtimes competing for the device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python glacier-engine_amd/build.py` "
                "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, res, args in _SIGS:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return [s[0] for s in _SIGS]


def ptr(a):
    """Raw address of a numpy array or a torch tensor (None -> NULL)."""
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    return a.data_ptr()


def check(rc, what, ctx=None):
    if rc != OK:
        msg = what
        if ctx is not None:
            err = lib().glacier_hip_last_error(ctx)
            if err:
                msg += f" ({err.decode()})"
        raise GlacierHipError(rc, msg)


# ---- synthetic generator (host) ------------------------------------------------------
def synth_int4(seed, tensor_id, nbytes):
    out = np.empty(nbytes, dtype=np.uint8)
    lib().glacier_hip_synth_int4(seed, tensor_id, ptr(out), nbytes)
    return out


def synth_scales_f16(seed, tensor_id, count, sigma=0.02):
    out = np.empty(count, dtype=np.uint16)
    lib().glacier_hip_synth_scales_f16(seed, tensor_id, sigma, ptr(out), count)
    return out


def synth_normal_f32(seed, tensor_id, count, sigma=0.02):
    out = np.empty(count, dtype=np.float32)
    lib().glacier_hip_synth_normal_f32(seed, tensor_id, sigma, ptr(out), count)
    return out


def synth_tokens(seed, tensor_id, vocab, count):
    out = np.empty(count, dtype=np.uint32)
    lib().glacier_hip_synth_tokens(seed, tensor_id, vocab, ptr(out), count)
    return out


def tensor_id(layer, which):
    return lib().glacier_hip_synth_tensor_id(layer, which)


GLOBAL_LAYER = 0xFFFFFF
# per-layer tensor slots used by glacier_hip_model_init_random
SLOT = dict(input_norm=0, post_attn_norm=1, wq=2, sq=3, wk=4, sk=5, wv=6, sv=7, wo=8, so=9,
            w_gate=10, s_gate=11, w_up=12, s_up=13, w_down=14, s_down=15,
            embedding=20, final_norm=21, lm_head=22, lm_head_scales=23)


def random_model_host(cfg, seed):
    """Host tensors identical to what glacier_hip_model_init_random uploads.

    Returns a dict with per-layer dicts (packed uint8 codes in the reference
    row-major layout, float32 scales that are exact fp16 values, f32 norms)
    and the global tensors."""
    D, F, V = cfg["dim"], cfg["hidden_dim"], cfg["vocab_size"]
    kvd = cfg["num_kv_heads"] * cfg["head_dim"]
    f16 = lambda a: a.view(np.float16).astype(np.float32)
    shapes = dict(q=(D, D), k=(kvd, D), v=(kvd, D), o=(D, D), gate=(F, D), up=(F, D),
                  down=(D, F))
    layers = []
    for l in range(cfg["num_layers"]):
        t = lambda which: tensor_id(l, which)
        L = dict(input_norm=synth_normal_f32(seed, t(0), D),
                 post_attn_norm=synth_normal_f32(seed, t(1), D))
        for i, name in enumerate(["q", "k", "v", "o", "gate", "up", "down"]):
            n, k = shapes[name]
            L["w_" + name] = synth_int4(seed, t(2 + 2 * i), n * k // 2)
            L["s_" + name] = f16(synth_scales_f16(seed, t(3 + 2 * i), n * k // 32))
        layers.append(L)
    G = GLOBAL_LAYER
    return dict(
        layers=layers,
        embedding=synth_normal_f32(seed, tensor_id(G, 20), V * D),
        final_norm=synth_normal_f32(seed, tensor_id(G, 21), D),
        lm_head=synth_int4(seed, tensor_id(G, 22), V * D // 2),
        lm_head_scales=f16(synth_scales_f16(seed, tensor_id(G, 23), V * D // 32)),
    )


class PageImageError(GlacierHipError):
    """A rejected page image or checkpoint restore; .reason is the
    reference's error name."""

    def __init__(self, code, reason, what):
        super().__init__(code, f"{what}: {reason}")
        self.reason = reason


def page_image_decode(image, challenge):
    """glacier_hip_page_image_decode -> PageImageInfo (PageImageError on rejection)."""
    info = PageImageInfo()
    buf = C.create_string_buffer(bytes(image), len(image))
    rc = lib().glacier_hip_page_image_decode(buf, len(image), bytes(challenge), C.byref(info))
    if rc != OK:
        raise PageImageError(rc, PAGE_IMAGE_ERRORS[info.error], "page_image_decode")
    return info


def page_image_encode_canonical(source_root, num_layers, dim, max_seq, source_ref, committed_rows,
                                payload, challenge):
    need = lib().glacier_hip_page_image_bytes(num_layers, dim, committed_rows) or 256
    out = C.create_string_buffer(need)
    n = C.c_uint64()
    info = PageImageInfo()
    buf = C.create_string_buffer(bytes(payload), len(payload))
    rc = lib().glacier_hip_page_image_encode_canonical(
        C.byref(source_root), num_layers, dim, max_seq, C.byref(source_ref), committed_rows, buf,
        len(payload), bytes(challenge), out, need, C.byref(n), C.byref(info))
    if rc != OK:
        raise PageImageError(rc, PAGE_IMAGE_ERRORS[info.error], "page_image_encode_canonical")
    return out.raw[:n.value]


class GlrtError(GlacierHipError):
    """A prepared runtime image that failed validation; .reason is the
    reference's error name."""

    def __init__(self, code, reason, what):
        super().__init__(code, f"{what}: {reason}")
        self.reason = reason


class GlrtImage:
    """A validated .glrt image (glacier_hip_glrt_open); host only."""

    def __init__(self, path, verify_payload_crc=True, verify_payload_digest=True, allow_v1=True,
                 expected_source=None):
        o = GlrtOpenOptions(verify_payload_crc=int(verify_payload_crc),
                            verify_payload_digest=int(verify_payload_digest),
                            allow_v1=int(allow_v1), check_source_fingerprint=int(expected_source is not None))
        if expected_source is not None:
            o.expected_source_fingerprint[:] = list(expected_source)
        self.info = GlrtInfo()
        h = _P()
        rc = lib().glacier_hip_glrt_open(os.fsencode(path), C.byref(o), C.byref(h), C.byref(self.info))
        if rc != OK:
            raise GlrtError(rc, GLRT_ERRORS[self.info.error], "glrt_open")
        self.h = h

    def record_at(self, i):
        r = GlrtRecord()
        check(lib().glacier_hip_glrt_record_at(self.h, i, C.byref(r)), "glrt_record_at")
        return r

    def records(self):
        return [self.record_at(i) for i in range(self.info.record_count)]

    def find(self, layer, kind, role=0):
        r = GlrtRecord()
        rc = lib().glacier_hip_glrt_find(self.h, layer, kind, role, C.byref(r))
        if rc == NOT_FOUND:
            return None
        check(rc, "glrt_find")
        return r

    def stream(self, record, s):
        p, n = _P(), C.c_uint64()
        check(lib().glacier_hip_glrt_stream(self.h, C.byref(record), s, C.byref(p), C.byref(n)),
              "glrt_stream")
        return C.string_at(p.value, n.value) if n.value else b""

    def identity(self):
        d, n = (C.c_uint8 * 32)(), C.c_uint64()
        check(lib().glacier_hip_glrt_identity(self.h, d, C.byref(n)), "glrt_identity")
        return bytes(d), n.value

    def close(self):
        if self.h:
            lib().glacier_hip_glrt_close(self.h)
            self.h = None


class GlacierError(GlacierHipError):
    """A `.glacier` container or qio payload the reader refused; .reason is
    the reference's error name."""

    def __init__(self, code, what):
        self.reason = GLACIER_ERRORS[code] if 0 <= code < len(GLACIER_ERRORS) else str(code)
        super().__init__(code, f"{what}: {self.reason}")


def _glac(rc, what):
    if rc != 0:
        raise GlacierError(rc, what)


class Glacier:
    """An admitted portable .glacier container (glacier_hip_glacier_open); host only."""

    def __init__(self, path):
        h = _P()
        _glac(lib().glacier_hip_glacier_open(os.fsencode(path), C.byref(h)), "glacier_open")
        self.h = h

    def header(self):
        x = GlacierHeader()
        _glac(lib().glacier_hip_glacier_header(self.h, C.byref(x)), "glacier_header")
        return x

    def page(self, i):
        x = GlacierPage()
        _glac(lib().glacier_hip_glacier_page(self.h, i, C.byref(x)), "glacier_page")
        return x

    def pages(self):
        return [self.page(i) for i in range(self.header().num_pages)]

    def metadata(self):
        p, n = _P(), C.c_uint64()
        _glac(lib().glacier_hip_glacier_metadata(self.h, C.byref(p), C.byref(n)), "glacier_metadata")
        return C.string_at(p.value, n.value) if n.value else b""

    def read_page(self, i, capacity=None):
        n = self.page(i).data_len if capacity is None else capacity
        buf = (C.c_uint8 * max(n, 1))()
        _glac(lib().glacier_hip_glacier_read_page(self.h, i, buf, n), "glacier_read_page")
        return bytes(buf)[:self.page(i).data_len]

    def read_page_f32(self, i):
        pg = self.page(i)
        out = np.zeros(max(pg.row_end - pg.row_start, 1), np.float32)
        n = C.c_uint64()
        _glac(lib().glacier_hip_glacier_read_page_f32(self.h, i, ptr(out), out.size, C.byref(n)),
              "glacier_read_page_f32")
        return out[:n.value]

    def validate_crcs(self, buffer_bytes=64 * 1024):
        _glac(lib().glacier_hip_glacier_validate_crcs(self.h, buffer_bytes), "glacier_validate_crcs")

    def identity(self):
        d, n = (C.c_uint8 * 32)(), C.c_uint64()
        _glac(lib().glacier_hip_glacier_identity(self.h, d, C.byref(n)), "glacier_identity")
        return bytes(d), n.value

    def source_fingerprint(self):
        d = (C.c_uint8 * 32)()
        _glac(lib().glacier_hip_glacier_source_fingerprint(self.h, d), "glacier_source_fingerprint")
        return bytes(d)

    def assemble(self):
        """The loader's host assembly: (error name, GlacierAssembly)."""
        a = GlacierAssembly()
        lib().glacier_hip_glacier_assemble(self.h, C.byref(a))
        return GLACIER_ERRORS[a.error], a

    def close(self):
        if self.h:
            lib().glacier_hip_glacier_close(self.h)
            self.h = None


def qio_encode_f32(src, precision, group_size):
    src = np.ascontiguousarray(src, dtype=np.float32)
    n = C.c_uint64()
    rc = lib().glacier_hip_qio_encode_f32(ptr(src) if src.size else None, src.size, precision,
                                          group_size, None, 0, C.byref(n))
    if rc != GLACIER_ERRORS.index("BufferTooSmall"):
        _glac(rc, "qio_encode_f32")
    buf = (C.c_uint8 * max(n.value, 1))()
    _glac(lib().glacier_hip_qio_encode_f32(ptr(src) if src.size else None, src.size, precision,
                                           group_size, buf, n.value, C.byref(n)), "qio_encode_f32")
    return bytes(buf)[:n.value]


def qio_decode_f32(payload):
    payload = bytes(payload)
    b = (C.c_uint8 * max(len(payload), 1)).from_buffer_copy(payload.ljust(1, b"\0"))
    n = C.c_uint64()
    rc = lib().glacier_hip_qio_decode_f32(b, len(payload), None, 0, C.byref(n))
    if rc != GLACIER_ERRORS.index("BufferTooSmall"):
        _glac(rc, "qio_decode_f32")
        return np.zeros(0, np.float32)
    out = np.zeros(max(n.value, 1), np.float32)
    _glac(lib().glacier_hip_qio_decode_f32(b, len(payload), ptr(out), out.size, C.byref(n)),
          "qio_decode_f32")
    return out[:n.value]


# ---- thin object wrappers -------------------------------------------------------------
class Context:
    def __init__(self, device=0):
        self.L = lib()
        self.h = self.L.glacier_hip_init(device)
        if not self.h:
            raise GlacierHipError(NO_DEVICE, "glacier_hip_init: " +
                                  (self.L.glacier_hip_last_error(None) or b"").decode())

    def close(self):
        if self.h:
            check(self.L.glacier_hip_deinit(self.h), "deinit", self.h)
            self.h = None

    def info(self):
        d = DeviceInfo()
        check(self.L.glacier_hip_device_info(self.h, C.byref(d)), "device_info", self.h)
        return d

    def sync(self):
        check(self.L.glacier_hip_synchronize(self.h), "synchronize", self.h)

    def weight(self, packed, scales, in_f, out_f, group=32):
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        if scales.dtype == np.uint16:
            w = self.L.glacier_hip_int4_weight_create_f16scales(
                self.h, ptr(packed), packed.size, ptr(scales), scales.size, group, in_f, out_f)
        else:
            scales = np.ascontiguousarray(scales, dtype=np.float32)
            w = self.L.glacier_hip_int4_weight_create(
                self.h, ptr(packed), packed.size, ptr(scales), scales.size, group, in_f, out_f)
        if not w:
            raise GlacierHipError(INVALID_ARGUMENT, "int4_weight_create: " +
                                  self.L.glacier_hip_last_error(self.h).decode())
        return w


class Model:
    def __init__(self, ctx, cfg):
        self.ctx = ctx
        self.cfg = dict(cfg)
        c = ModelConfig(**{k: cfg[k] for k, _ in ModelConfig._fields_})
        self.h = lib().glacier_hip_model_create(ctx.h, C.byref(c))
        if not self.h:
            raise GlacierHipError(INVALID_ARGUMENT, "model_create: " +
                                  lib().glacier_hip_last_error(ctx.h).decode())

    def init_random(self, seed):
        check(lib().glacier_hip_model_init_random(self.h, seed), "model_init_random", self.ctx.h)

    def set_from_host(self, host):
        for l, L in enumerate(host["layers"]):
            keep = {k: np.ascontiguousarray(v) for k, v in L.items()}
            lh = LayerHost(
                input_norm=ptr(keep["input_norm"]), post_attn_norm=ptr(keep["post_attn_norm"]),
                wq=ptr(keep["w_q"]), wk=ptr(keep["w_k"]), wv=ptr(keep["w_v"]), wo=ptr(keep["w_o"]),
                w_gate=ptr(keep["w_gate"]), w_up=ptr(keep["w_up"]), w_down=ptr(keep["w_down"]),
                sq=ptr(keep["s_q"]), sk=ptr(keep["s_k"]), sv=ptr(keep["s_v"]), so=ptr(keep["s_o"]),
                s_gate=ptr(keep["s_gate"]), s_up=ptr(keep["s_up"]), s_down=ptr(keep["s_down"]),
                bq=ptr(keep.get("bq")), bk=ptr(keep.get("bk")), bv=ptr(keep.get("bv")))
            check(lib().glacier_hip_model_set_layer(self.h, l, C.byref(lh)), "set_layer", self.ctx.h)
        check(lib().glacier_hip_model_set_globals(
            self.h, ptr(host["embedding"]), ptr(host["final_norm"]), ptr(host["lm_head"]),
            ptr(np.ascontiguousarray(host["lm_head_scales"], dtype=np.float32))),
            "set_globals", self.ctx.h)

    @classmethod
    def load_glrt(cls, ctx, image):
        """glacier_hip_model_load_glrt: a device model from a validated image."""
        m = cls.__new__(cls)
        m.ctx = ctx
        i = image.info
        m.cfg = dict(num_layers=i.layers, dim=i.dim, hidden_dim=i.hidden_dim, num_heads=i.heads,
                     num_kv_heads=i.kv_heads, head_dim=i.head_dim, vocab_size=i.vocab,
                     group_size=32, rms_eps=i.rms_eps, rope_theta=i.rope_theta)
        m.report = GlrtLoadReport()
        m.h = lib().glacier_hip_model_load_glrt(ctx.h, image.h, C.byref(m.report))
        if not m.h:
            raise GlrtError(INVALID_ARGUMENT, GLRT_ERRORS[m.report.error], "model_load_glrt")
        return m

    @classmethod
    def load_glacier(cls, ctx, container, override=None, tie_word_embeddings=False):
        """glacier_hip_model_load_glacier: a device model from an admitted
        .glacier container; `override` holds ModelConfig fields (zero or
        absent: the page geometry and the reference's defaults)."""
        m = cls.__new__(cls)
        m.ctx = ctx
        o = ModelConfig(**(override or {}))
        m.report = GlacierLoadReport()
        m.h = lib().glacier_hip_model_load_glacier(ctx.h, container.h, C.byref(o),
                                                   int(tie_word_embeddings), C.byref(m.report))
        if not m.h:
            raise GlacierError(m.report.error, "model_load_glacier")
        c = m.report.config
        m.cfg = {k: getattr(c, k) for k, _ in ModelConfig._fields_}
        return m

    def weight_bytes(self):
        return lib().glacier_hip_model_weight_bytes(self.h)

    def close(self):
        if self.h:
            lib().glacier_hip_model_destroy(self.h)
            self.h = None


class Session:
    def __init__(self, model, max_lanes, max_positions, kv_dtype=F32, total_pages=0,
                 layer_activation=ACT_AUTO, head_activation=ACT_AUTO, use_graph=True,
                 prefill_chunk=0, split_attention_o=False):
        self.model = model
        self.max_lanes = max_lanes
        o = SessionOptions(max_lanes=max_lanes, max_positions=max_positions,
                           total_pages=total_pages, kv_dtype=kv_dtype,
                           layer_activation=layer_activation, head_activation=head_activation,
                           use_graph=int(use_graph), prefill_chunk=prefill_chunk,
                           split_attention_o=1 if split_attention_o else 0)
        self.h = lib().glacier_hip_session_create(model.h, C.byref(o))
        if not self.h:
            raise GlacierHipError(INVALID_ARGUMENT, "session_create: " +
                                  lib().glacier_hip_last_error(model.ctx.h).decode())
        self.vocab = model.cfg["vocab_size"]

    def begin(self, lane, seed=0):
        check(lib().glacier_hip_session_lane_begin(self.h, lane, seed), "lane_begin")

    def prefill(self, lane, tokens, want_logits=False):
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        first = np.zeros(1, dtype=np.uint32)
        logits = np.empty(self.vocab, dtype=np.float32) if want_logits else None
        rc = lib().glacier_hip_session_prefill(self.h, lane, ptr(toks), toks.size, ptr(first),
                                               ptr(logits))
        check(rc, "prefill", self.model.ctx.h)
        return (int(first[0]), logits) if want_logits else int(first[0])

    def step(self, lanes, tokens, eligible=None, want_logits=False, raise_on_error=True):
        lanes = np.ascontiguousarray(lanes, dtype=np.uint32)
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        nxt = np.zeros(lanes.size, dtype=np.uint32)
        logits = np.empty((lanes.size, self.vocab), dtype=np.float32) if want_logits else None
        el = None if eligible is None else np.ascontiguousarray(eligible, dtype=np.uint64)
        rc = lib().glacier_hip_session_decode_step(self.h, ptr(lanes), ptr(toks), lanes.size,
                                                   ptr(el), ptr(nxt), ptr(logits))
        if raise_on_error:
            check(rc, "decode_step", self.model.ctx.h)
            return (nxt, logits) if want_logits else nxt
        return rc, nxt

    def root(self, lane):
        r = PageMapRoot()
        check(lib().glacier_hip_session_lane_root(self.h, lane, C.byref(r)), "lane_root")
        return r

    def state(self, lane):
        s = LaneState()
        check(lib().glacier_hip_session_lane_state(self.h, lane, C.byref(s)), "lane_state")
        return s

    def kv_sha256(self, lane):
        out = (C.c_uint8 * 32)()
        check(lib().glacier_hip_session_lane_kv_sha256(self.h, lane, out), "kv_sha256")
        return bytes(out)

    def kv_row(self, lane, layer, value, pos, kv_dim):
        out = np.empty(kv_dim, dtype=np.float32)
        check(lib().glacier_hip_session_read_kv_row(self.h, lane, layer, value, pos, ptr(out)),
              "read_kv_row")
        return out

    def page_of(self, lane, logical_page):
        v = C.c_int32()
        check(lib().glacier_hip_session_page_of(self.h, lane, logical_page, C.byref(v)), "page_of")
        return v.value

    def prefill_staged(self, lane, tokens):
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        first = np.zeros(1, dtype=np.uint32)
        check(lib().glacier_hip_session_prefill_staged(self.h, lane, ptr(toks), toks.size,
                                                       ptr(first), None),
              "prefill_staged", self.model.ctx.h)
        return int(first[0])

    def step_prepare(self, lanes, tokens, binding, eligible=None):
        """Returns (rc, proposal, proposal_sha256 bytes, next tokens)."""
        lanes = np.ascontiguousarray(lanes, dtype=np.uint32)
        toks = np.ascontiguousarray(tokens if tokens is not None else np.zeros(lanes.size),
                                    dtype=np.uint32)
        nxt = np.zeros(lanes.size, dtype=np.uint32)
        el = None if eligible is None else np.ascontiguousarray(eligible, dtype=np.uint64)
        prop = TokenProposal()
        sha = (C.c_uint8 * 32)()
        rc = lib().glacier_hip_session_step_prepare(self.h, ptr(lanes), ptr(toks), lanes.size,
                                                    ptr(el), C.byref(binding), C.byref(prop),
                                                    sha, ptr(nxt), None)
        return rc, prop, bytes(sha), nxt

    def step_prepare_v3(self, lanes, tokens, binding, terminal_reason=None, eligible=None):
        """A wave of leased lanes of one cohort sealed as ProposalV3.
        terminal_reason[i]: 0, or 1 + TERMINAL_* of lane i's token. Returns
        (rc, proposal, proposal_sha256 bytes, next tokens)."""
        lanes = np.ascontiguousarray(lanes, dtype=np.uint32)
        toks = np.ascontiguousarray(tokens if tokens is not None else np.zeros(lanes.size),
                                    dtype=np.uint32)
        reasons = None if terminal_reason is None else \
            np.ascontiguousarray(terminal_reason, dtype=np.uint32)
        nxt = np.zeros(lanes.size, dtype=np.uint32)
        el = None if eligible is None else np.ascontiguousarray(eligible, dtype=np.uint64)
        prop = TokenProposalV3()
        sha = (C.c_uint8 * 32)()
        rc = lib().glacier_hip_session_step_prepare_v3(self.h, ptr(lanes), ptr(toks), lanes.size,
                                                       ptr(el), C.byref(binding), ptr(reasons),
                                                       C.byref(prop), sha, ptr(nxt))
        return rc, prop, bytes(sha), nxt

    def step_commit(self, ack):
        rec = CommitReceipt()
        rc = lib().glacier_hip_session_step_commit(self.h, C.byref(ack), C.byref(rec))
        return rc, rec

    def step_abort(self):
        return lib().glacier_hip_session_step_abort(self.h)

    def page_generation(self, lane, logical_page):
        v = C.c_uint64()
        check(lib().glacier_hip_session_page_generation(self.h, lane, logical_page, C.byref(v)),
              "page_generation")
        return v.value

    def set_head_domain(self, mode):
        check(lib().glacier_hip_session_set_head_domain(self.h, mode), "set_head_domain")

    def inject_failure(self, enable):
        check(lib().glacier_hip_session_inject_failure(self.h, 1 if enable else 0), "inject")

    def trace_layers(self, enable):
        check(lib().glacier_hip_session_trace_layers(self.h, 1 if enable else 0), "trace_layers")

    PROBE = dict(qkv=0, attention=1, o=2, gate_up=3, down=4)

    def probe_kernel(self, kind):
        """Time one in-token launch per layer with HIP events (kind: a PROBE
        key, or None to stop); resets the totals."""
        check(lib().glacier_hip_session_probe_kernel(self.h, -1 if kind is None
                                                     else self.PROBE[kind]), "probe_kernel")

    def probe_replay(self, kind, reps=4):
        """Average microseconds of the last step's `kind` (gate_up / down)
        launches replayed back to back over every layer."""
        us = C.c_double()
        check(lib().glacier_hip_session_probe_replay(self.h, self.PROBE[kind], reps, C.byref(us)),
              "probe_replay", self.model.ctx.h)
        return us.value

    def probe_read(self):
        """(total microseconds, launches) since the last probe_kernel."""
        us, n = C.c_double(), C.c_uint64()
        check(lib().glacier_hip_session_probe_read(self.h, C.byref(us), C.byref(n)), "probe_read")
        return us.value, n.value

    def layer_trace(self):
        """The last traced step's residual after every layer: [num_layers, rows, dim]."""
        c = self.model.cfg
        buf = np.zeros(c["num_layers"] * self.max_lanes * c["dim"], np.float32)
        rows = C.c_uint32()
        check(lib().glacier_hip_session_layer_trace(self.h, buf.ctypes.data, C.byref(rows)),
              "layer_trace")
        n = rows.value
        return buf[:c["num_layers"] * n * c["dim"]].reshape(c["num_layers"], n, c["dim"])

    def encode_page_image(self, lane, logical_page, challenge):
        """glacier_hip_session_encode_page_image -> (image bytes, PageImageInfo)."""
        cfg = self.model.cfg
        need = lib().glacier_hip_page_image_bytes(cfg["num_layers"],
                                                  cfg["num_kv_heads"] * cfg["head_dim"], 16)
        out = C.create_string_buffer(need)
        n = C.c_uint64()
        info = PageImageInfo()
        rc = lib().glacier_hip_session_encode_page_image(self.h, lane, logical_page, bytes(challenge),
                                                         out, need, C.byref(n), C.byref(info))
        if rc != OK:
            if rc == INVALID_CHECKPOINT:
                raise PageImageError(rc, PAGE_IMAGE_ERRORS[info.error], "encode_page_image")
            check(rc, "encode_page_image", self.model.ctx.h)
        return out.raw[:n.value], info

    def restore_checkpoint(self, lane, images, challenge, seed=0):
        """glacier_hip_session_restore_checkpoint -> (CheckpointRestore, target refs)."""
        n = len(images)
        arr = (C.c_char_p * n)(*[bytes(i) for i in images])
        lens = (C.c_uint64 * n)(*[len(i) for i in images])
        out = CheckpointRestore()
        refs = (PageRef * max(n, 1))()
        rc = lib().glacier_hip_session_restore_checkpoint(self.h, lane, arr, lens, n,
                                                          bytes(challenge), seed, C.byref(out), refs)
        if rc != OK:
            if rc == INVALID_CHECKPOINT:
                raise PageImageError(rc, PAGE_IMAGE_ERRORS[out.error], "restore_checkpoint")
            check(rc, "restore_checkpoint", self.model.ctx.h)
        return out, [refs[i] for i in range(n)]

    def close(self):
        if self.h:
            lib().glacier_hip_session_destroy(self.h)
            self.h = None


class KvPages:
    """Host page map of one paged KV cache (glacier_hip_kv_pages_*): the
    reference's PagedKVCache row transaction without a device."""

    def __init__(self, num_layers, kv_dim, max_seq, pool_pages):
        self.h = lib().glacier_hip_kv_pages_create(num_layers, kv_dim, max_seq, pool_pages)
        if not self.h:
            raise GlacierHipError(INVALID_ARGUMENT, "kv_pages_create")

    def begin_row(self):
        m = RowTxnMark()
        rc = lib().glacier_hip_kv_pages_begin_row(self.h, C.byref(m))
        return rc, m

    def commit_row(self, mark):
        return lib().glacier_hip_kv_pages_commit_row(self.h, C.byref(mark))

    def abort_row(self, mark):
        return lib().glacier_hip_kv_pages_abort_row(self.h, C.byref(mark))

    def staged_roots(self, mark):
        b, a = PageMapRoot(), PageMapRoot()
        rc = lib().glacier_hip_kv_pages_staged_root(self.h, C.byref(mark), C.byref(b), C.byref(a))
        return rc, b, a

    def reset(self):
        return lib().glacier_hip_kv_pages_reset(self.h)

    def root(self):
        r = PageMapRoot()
        check(lib().glacier_hip_kv_pages_root(self.h, C.byref(r)), "kv_pages_root")
        return r

    def page(self, logical_page):
        p, g = C.c_int32(), C.c_uint64()
        check(lib().glacier_hip_kv_pages_page(self.h, logical_page, C.byref(p), C.byref(g)),
              "kv_pages_page")
        return p.value, g.value

    def validate_page_ref(self, ref):
        return lib().glacier_hip_kv_pages_validate_page_ref(self.h, C.byref(ref))

    def ledger(self):
        led = ResidentLedger()
        check(lib().glacier_hip_kv_pages_ledger(self.h, C.byref(led)), "kv_pages_ledger")
        return {n: getattr(led, n) for n, _ in ResidentLedger._fields_}

    def page_count(self):
        return self.ledger()["page_count_capacity"]

    def kv_sha256(self):
        b = (C.c_uint8 * 32)()
        check(lib().glacier_hip_kv_pages_kv_sha256(self.h, b), "kv_pages_kv_sha256")
        return bytes(b)

    def is_retired(self):
        v = C.c_int32()
        check(lib().glacier_hip_kv_pages_is_retired(self.h, C.byref(v)), "kv_pages_is_retired")
        return bool(v.value)

    def set_pool_capacity(self, pages):
        return lib().glacier_hip_kv_pages_set_pool_capacity(self.h, pages)

    def close(self):
        if self.h:
            lib().glacier_hip_kv_pages_destroy(self.h)
            self.h = None

    __del__ = close


STALE_HANDLE, NO_RUNNABLE, INCOMPLETE_DRAIN, SCHEDULER_CLOSED, SCHEDULER_POISONED = 15, 16, 17, 18, 19
SERVICE_IN_FLIGHT, STALE_SERVICE_PERMIT, SINK_REJECTED = 23, 24, 25


def _claim(d):
    c = Claim()
    for k, v in (d or {}).items():
        setattr(c, k, v)
    return c


class LaneWeave:
    """Python face of glacier_hip_lane_weave_* (host scheduler; no GPU)."""

    def __init__(self, capacity, bank_limits=None, bank_epoch=1, scheduler_epoch=1,
                 challenge=None, max_weight=64, max_projection_quanta=1_000_000,
                 max_projection_operations=1_000_000):
        lim = Limits(*([2**64 - 1] * 11))
        for k, v in (bank_limits or {}).items():
            setattr(lim, k, v)
        ch = (C.c_uint8 * 32)(*(challenge or (bytes([0xA5]) + bytes(31))))
        self.h = lib().glacier_hip_lane_weave_create(capacity, C.byref(lim), bank_epoch,
                                                     scheduler_epoch, ch, max_weight,
                                                     max_projection_quanta,
                                                     max_projection_operations)
        if not self.h:
            raise GlacierHipError(INVALID_ARGUMENT, "lane_weave_create")

    def close_handle(self):
        if self.h:
            lib().glacier_hip_lane_weave_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close_handle()
        except Exception:
            pass

    @staticmethod
    def spec(tenant_key, request_key, request_generation, resource_owner_key, weight,
             work_quanta, deadline_tick, claim):
        return RequestSpec(tenant_key, request_key, request_generation, resource_owner_key,
                           weight, work_quanta, deadline_tick, _claim(claim))

    def admit(self, spec):
        ok, h, e = C.c_int(0), LaneHandle(), LaneEvent()
        check(lib().glacier_hip_lane_weave_admit(self.h, C.byref(spec), C.byref(ok), C.byref(h),
                                                 C.byref(e)), "lane_weave_admit")
        return bool(ok.value), (h if ok.value else None), e

    def _ev(self, fn, *args):
        e = LaneEvent()
        rc = fn(self.h, *args, C.byref(e))
        return rc, e

    def serve_one(self):
        rc, e = self._ev(lib().glacier_hip_lane_weave_serve_one)
        check(rc, "lane_weave_serve_one")
        return e

    def plan_wave(self, max_count):
        out = (C.c_uint32 * max(1, max_count))()
        n = C.c_uint32(0)
        check(lib().glacier_hip_lane_weave_plan_wave(self.h, max_count, out, C.byref(n)),
              "lane_weave_plan_wave")
        return [int(out[i]) for i in range(n.value)]

    def retire(self, handle):
        return self._ev(lib().glacier_hip_lane_weave_retire, C.byref(handle))

    def cancel(self, handle):
        return self._ev(lib().glacier_hip_lane_weave_cancel, C.byref(handle))

    def close(self):
        return self._ev(lib().glacier_hip_lane_weave_close)

    def slot(self, i):
        h, st, rem = LaneHandle(), C.c_uint32(), C.c_uint64()
        check(lib().glacier_hip_lane_weave_slot(self.h, i, C.byref(h), C.byref(st),
                                                C.byref(rem)), "lane_weave_slot")
        return h, int(st.value), int(rem.value)

    def wave(self, sess, lane_of_slot, tokens_by_lane, eligible_by_lane=None, max_count=None):
        """One decode wave through glacier_hip_session_lane_weave_wave.
        tokens_by_lane (uint32 array) is updated in place; returns
        (slots, events)."""
        los = np.ascontiguousarray(lane_of_slot, dtype=np.uint32)
        mc = max_count or len(los)
        slots = np.zeros(mc, dtype=np.uint32)
        evs = (LaneEvent * mc)()
        n = C.c_uint32(0)
        rc = lib().glacier_hip_session_lane_weave_wave(sess.h, self.h, ptr(los), los.size,
                                                       ptr(tokens_by_lane), ptr(eligible_by_lane),
                                                       mc, ptr(slots), evs, C.byref(n))
        check(rc, "lane_weave_wave", sess.model.ctx.h)
        return slots[:n.value].tolist(), [evs[i] for i in range(n.value)]

    def chain_head(self):
        out = (C.c_uint8 * 32)()
        check(lib().glacier_hip_lane_weave_chain_head(self.h, out), "chain_head")
        return bytes(out)

    def prepare_service(self):
        """prepareService -> (rc, ServicePermit)."""
        p = ServicePermit()
        rc = lib().glacier_hip_lane_weave_prepare_service(self.h, C.byref(p))
        return rc, p

    def commit_service(self, permit):
        """commitService -> (rc, event)."""
        return self._ev(lib().glacier_hip_lane_weave_commit_service, C.byref(permit))

    def abort_service(self, permit):
        return lib().glacier_hip_lane_weave_abort_service(self.h, C.byref(permit))

    def state_sha256(self):
        out = (C.c_uint8 * 32)()
        check(lib().glacier_hip_lane_weave_state_sha256(self.h, out), "state_sha256")
        return bytes(out)

    def wave_staged(self, sess, lane_of_slot, tokens_by_lane, sink, eligible_by_lane=None,
                    max_count=None):
        """glacier_hip_session_lane_weave_wave_staged; sink(stages) returns
        True to acknowledge the wave's stages (a list of WaveStage copies).
        Returns (rc, slots, events)."""
        los = np.ascontiguousarray(lane_of_slot, dtype=np.uint32)
        mc = max_count or len(los)
        slots = np.zeros(mc, dtype=np.uint32)
        evs = (LaneEvent * mc)()
        n = C.c_uint32(0)

        def cb(_ctx, stages, count):
            return 0 if sink([WaveStage.from_buffer_copy(stages[i]) for i in range(count)]) else 1

        fn = WAVE_SINK(cb)
        rc = lib().glacier_hip_session_lane_weave_wave_staged(
            sess.h, self.h, ptr(los), los.size, ptr(tokens_by_lane), ptr(eligible_by_lane), mc, fn,
            None, ptr(slots), evs, C.byref(n))
        return rc, slots[:n.value].tolist(), [evs[i] for i in range(n.value)]


class LeaseError(Exception):
    """A lease verb's status, by the reference's error name (e.g. 'InvalidBinding')."""

    def __init__(self, code, what):
        self.code = code
        self.reason = LEASE_STATUS[code] if 0 <= code < len(LEASE_STATUS) else f"status {code}"
        super().__init__(f"{what}: {self.reason}")


def lease_check(rc, what):
    if rc != 0:
        raise LeaseError(rc, what)


def make_claim(**kw):
    c = Claim()
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def make_limits(**kw):
    lim = Limits(*([2**64 - 1] * len(Limits._fields_)))
    for k, v in kw.items():
        setattr(lim, k, v)
    return lim


class LeaseBank:
    """ResourceBank receipts with LeaseTree page ownership (glacier_hip_lease_*)."""

    def __init__(self, slots, nodes, epoch, **limits):
        self.h = lib().glacier_hip_lease_bank_create(slots, nodes, C.byref(make_limits(**limits)),
                                                     epoch)
        if not self.h:
            raise LeaseError(1, "lease_bank_create")

    def reserve(self, owner_key, **claim):
        r = BankReceipt()
        lease_check(lib().glacier_hip_lease_bank_reserve(self.h, owner_key,
                                                         C.byref(make_claim(**claim)), C.byref(r)),
                    "reserve")
        return r

    def commit(self, reservation):
        r = BankReceipt()
        lease_check(lib().glacier_hip_lease_bank_commit(self.h, C.byref(reservation), C.byref(r)),
                    "commit")
        return r

    def release(self, receipt):
        lease_check(lib().glacier_hip_lease_bank_release(self.h, C.byref(receipt)), "release")

    def open_tree(self, receipt, tree_key, authority_key, **ceiling):
        t = LeaseTree()
        lease_check(lib().glacier_hip_lease_tree_open(self.h, C.byref(receipt), tree_key,
                                                      authority_key, C.byref(make_claim(**ceiling)),
                                                      C.byref(t)), "open_tree")
        return t

    def open_scope(self, tree, scope_key, tenant_key, **ceiling):
        """Adds a scope; `tree` (a LeaseTree) is replaced in place."""
        n = LeaseNode()
        lease_check(lib().glacier_hip_lease_scope_open(self.h, C.byref(tree), scope_key, tenant_key,
                                                       C.byref(make_claim(**ceiling)), C.byref(n)),
                    "open_scope")
        return n

    def close_tree(self, tree):
        lease_check(lib().glacier_hip_lease_tree_close(self.h, C.byref(tree)), "close_tree")

    def validate_tree(self, tree):
        return lib().glacier_hip_lease_tree_validate(self.h, C.byref(tree))

    def bind_session(self, tree, request_epoch, session_id):
        lease_check(lib().glacier_hip_lease_session_bind(self.h, C.byref(tree), request_epoch,
                                                         session_id), "bind_session")

    def close_session(self, receipt, request_epoch, session_id, next_sequence):
        lease_check(lib().glacier_hip_lease_session_close(self.h, C.byref(receipt), request_epoch,
                                                          session_id, next_sequence),
                    "close_session")

    def begin_publication(self, tree, request_epoch, session_id, expected_sequence):
        p = PublicationPermit()
        lease_check(lib().glacier_hip_lease_publication_begin(
            self.h, C.byref(tree), request_epoch, session_id, expected_sequence, C.byref(p)),
            "begin_publication")
        return p

    def commit_publication(self, permit):
        lease_check(lib().glacier_hip_lease_publication_commit(self.h, C.byref(permit)),
                    "commit_publication")

    def abort_publication(self, permit):
        lease_check(lib().glacier_hip_lease_publication_abort(self.h, C.byref(permit)),
                    "abort_publication")

    def snapshot(self):
        s = LeaseBankSnapshot()
        lease_check(lib().glacier_hip_lease_bank_snapshot(self.h, C.byref(s)), "snapshot")
        out = {n: getattr(s, n) for n, _ in LeaseBankSnapshot._fields_[2:]}
        out["used"] = {n: getattr(s.used, n) for n in CLAIM_FIELDS}
        out["peak"] = {n: getattr(s.peak, n) for n in CLAIM_FIELDS}
        return out

    def close(self):
        if self.h:
            lib().glacier_hip_lease_bank_destroy(self.h)
            self.h = None

    __del__ = close


class LeasedKV:
    """One lane's page map leased through a LeaseTree (glacier_hip_leased_kv_*).
    `tree` and `sequence` are the cohort's shared cells (a LeaseTree and a
    ctypes c_uint64); `bindings` is created here, one entry per logical page."""

    def __init__(self, bank, tree, scope, target, request_epoch, session_id, sequence, lane=None,
                 binding_count=None):
        self.bank, self.tree, self.sequence, self.target = bank, tree, sequence, target
        self.scope = scope
        n = binding_count if binding_count is not None else target.page_count()
        self.bindings = (PageLeaseBinding * max(n, 1))()
        self.h = _P()
        if lane is None:
            rc = lib().glacier_hip_leased_kv_create(bank.h, C.byref(tree), C.byref(scope), target.h,
                                                    self.bindings, n, request_epoch, session_id,
                                                    C.byref(sequence), C.byref(self.h))
        else:
            rc = lib().glacier_hip_leased_kv_create_for_lane(
                bank.h, C.byref(tree), C.byref(scope), target.h, lane, self.bindings, n,
                request_epoch, session_id, C.byref(sequence), C.byref(self.h))
        lease_check(rc, "leased_kv_create")

    def plan_next_row(self):
        p = LeasedRowPlan()
        lease_check(lib().glacier_hip_leased_kv_plan_next_row(self.h, C.byref(p)), "plan_next_row")
        return p

    def begin_row(self, plan):
        t = LeasedRowTxn()
        lease_check(lib().glacier_hip_leased_kv_begin_row(self.h, C.byref(plan), C.byref(t)),
                    "begin_row")
        return t

    def commit_row(self, txn):
        r = PageMapRoot()
        lease_check(lib().glacier_hip_leased_kv_commit_row(self.h, C.byref(txn), C.byref(r)),
                    "commit_row")
        return r

    def abort_row(self, txn):
        lease_check(lib().glacier_hip_leased_kv_abort_row(self.h, C.byref(txn)), "abort_row")

    def append_row(self, txn, layer, k, v):
        kk = (C.c_float * len(k))(*k)
        vv = (C.c_float * len(v))(*v)
        check(lib().glacier_hip_kv_pages_append_row(self.target.h, C.byref(txn.mark), layer, kk, vv),
              "append_row")

    def binding_summary(self):
        s = BindingSummary()
        lease_check(lib().glacier_hip_leased_kv_binding_summary(self.h, C.byref(s)),
                    "binding_summary")
        return s

    def allocation_set(self):
        a = AllocationSet()
        lease_check(lib().glacier_hip_leased_kv_allocation_set(self.h, C.byref(a)),
                    "allocation_set")
        return a

    def lifecycle(self):
        v = C.c_uint32()
        lease_check(lib().glacier_hip_leased_kv_lifecycle(self.h, C.byref(v)), "lifecycle")
        return ["live", "terminal_retained", "freed_pending_uncharge", "reclaimed"][v.value]

    def root(self):
        r = PageMapRoot()
        lease_check(lib().glacier_hip_leased_kv_root(self.h, C.byref(r)), "root")
        return r

    def kv_sha256(self):
        b = (C.c_uint8 * 32)()
        lease_check(lib().glacier_hip_leased_kv_kv_sha256(self.h, b), "kv_sha256")
        return bytes(b)

    def seal_terminal(self, root, kv_sha256, sequence, reason, token):
        s = TerminalSeal()
        kv = (C.c_uint8 * 32)(*kv_sha256)
        lease_check(lib().glacier_hip_leased_kv_seal_terminal(self.h, C.byref(root), kv, sequence,
                                                              reason, token, C.byref(s)),
                    "seal_terminal")
        return s

    def begin_reclaim(self, seal, expected_sequence):
        f = FreedPayload()
        lease_check(lib().glacier_hip_leased_kv_begin_reclaim(self.h, C.byref(seal),
                                                              expected_sequence, C.byref(f)),
                    "begin_reclaim")
        return f

    def commit_reclaim(self, freed):
        r = ReclaimReceipt()
        lease_check(lib().glacier_hip_leased_kv_commit_reclaim(self.h, C.byref(freed), C.byref(r)),
                    "commit_reclaim")
        return r

    def terminal_seal(self):
        s = TerminalSeal()
        p, c = (C.c_uint8 * 32)(), (C.c_uint8 * 32)()
        lease_check(lib().glacier_hip_leased_kv_terminal_seal(self.h, C.byref(s), p, c),
                    "terminal_seal")
        return s, bytes(p), bytes(c)

    def reclaim_for_teardown(self, expected_sequence):
        lease_check(lib().glacier_hip_leased_kv_reclaim_for_teardown(self.h, expected_sequence),
                    "reclaim_for_teardown")

    def close(self):
        if self.h:
            lib().glacier_hip_leased_kv_destroy(self.h)
            self.h = None

    __del__ = close
