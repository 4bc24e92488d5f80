"""ctypes binding of libzs.so (include/zs.h).

This module only loads the library and declares the C structs; it raises if
the HIP library is missing -- there is no CPU fallback anywhere in the product.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libzs.so")

ZS_OK = 0
ZS_EINVAL = -1
ZS_EHIP = -2
ZS_ENOMEM = -3
ZS_ELIMIT = -4

ZS_ROW_MASKED = 1
ZS_ROW_LOGPROBS = 2
ZS_ROW_UNCERTAINTY = 4

ZS_SPEC_BACKGROUND = 1

ZS_ST_GREEDY = 1
ZS_ST_NONFINITE = 2
ZS_ST_SMALL = 4
ZS_ST_TOPLP_AMBIG = 8
ZS_ST_LIMIT = 0x100
ZS_ST_FALLBACK = 0x200



class RowParams(C.Structure):
    _fields_ = [
        ("temperature", C.c_float),
        ("top_k", C.c_uint32),
        ("top_p", C.c_float),
        ("min_p", C.c_float),
        ("repeat", C.c_float),
        ("presence", C.c_float),
        ("frequency", C.c_float),
        ("top_logprobs", C.c_uint32),
        ("flags", C.c_uint32),
        ("pad", C.c_uint32),
    ]


class Batch(C.Structure):
    _fields_ = [
        ("B", C.c_uint32),
        ("V", C.c_uint32),
        ("ld", C.c_uint64),
        ("d_logits", C.c_void_p),
        ("d_params", C.c_void_p),
        ("d_cnt_off", C.c_void_p),
        ("d_cnt_ids", C.c_void_p),
        ("d_cnt_vals", C.c_void_p),
        ("d_bias_off", C.c_void_p),
        ("d_bias_ids", C.c_void_p),
        ("d_bias_vals", C.c_void_p),
        ("d_ban_off", C.c_void_p),
        ("d_ban_ids", C.c_void_p),
        ("d_allow_bits", C.c_void_p),
        ("allow_words", C.c_uint32),
        ("top_stride", C.c_uint32),
        ("d_seed", C.c_void_p),
        ("d_counter", C.c_void_p),
        ("d_token", C.c_void_p),
        ("d_logprob", C.c_void_p),
        ("d_top_ids", C.c_void_p),
        ("d_top_lps", C.c_void_p),
        ("d_top_n", C.c_void_p),
        ("d_entropy", C.c_void_p),
        ("d_max_prob", C.c_void_p),
        ("d_margin", C.c_void_p),
        ("d_chosen_lp", C.c_void_p),
        ("d_status", C.c_void_p),
        ("pass_event", C.c_void_p),
    ]


class SpecBatch(C.Structure):
    _fields_ = [
        ("B", C.c_uint32), ("V", C.c_uint32), ("k", C.c_uint32),
        ("ld", C.c_uint64),
        ("d_target", C.c_void_p), ("d_draft", C.c_void_p), ("d_draft_ids", C.c_void_p),
        ("d_temperature", C.c_void_p), ("d_seed", C.c_void_p), ("d_counter", C.c_void_p),
        ("d_accepted", C.c_void_p), ("d_next", C.c_void_p), ("flags", C.c_uint32),
    ]


class LaneStream(C.Structure):
    _fields_ = [("temp", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float), ("base_seed", C.c_uint32),
                ("gen_index", C.c_uint32)]


class HallucReport(C.Structure):
    _fields_ = [("risk_score", C.c_float), ("mean_entropy", C.c_float), ("normalized_entropy", C.c_float),
                ("risky_fraction", C.c_float), ("peak_token", C.c_int64), ("n_tokens", C.c_uint64)]


# name -> (restype, argtypes); every symbol include/zs.h declares
SIGNATURES = {
    "zs_abi_version": (C.c_int, []),
    "zs_struct_layout": (C.c_int, [C.c_int, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t), C.c_size_t]),
    "zs_ctx_create": (C.c_int, [C.c_int, C.c_uint32, C.c_uint32, C.POINTER(C.c_void_p)]),
    "zs_ctx_destroy": (None, [C.c_void_p]),
    "zs_last_error": (C.c_char_p, [C.c_void_p]),
    "zs_vocab_create": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32,
                                  C.POINTER(C.c_void_p)]),
    "zs_vocab_destroy": (None, [C.c_void_p]),
    "zs_dfa_create": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p,
                                C.POINTER(C.c_void_p)]),
    "zs_dfa_destroy": (None, [C.c_void_p]),
    "zs_dfa_is_live": (C.c_int, [C.c_void_p, C.c_uint32]),
    "zs_dfa_is_accept": (C.c_int, [C.c_void_p, C.c_uint32]),
    "zs_dfa_advance": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.POINTER(C.c_uint32),
                                 C.POINTER(C.c_int)]),
    "zs_dfa_mask": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32,
                              C.c_void_p, C.c_void_p, C.c_void_p]),
    "zs_dfa_memo_clear": (None, [C.c_void_p]),
    "zs_dfa_table_form": (C.c_int, [C.c_void_p]),
    "zs_sample": (C.c_int, [C.c_void_p, C.POINTER(Batch), C.c_void_p]),
    "zs_set_profiling": (C.c_int, [C.c_void_p, C.c_int]),
    "zs_spec_verify": (C.c_int, [C.c_void_p, C.POINTER(SpecBatch), C.c_void_p]),
    "zs_spec_verify_static": (C.c_int, [C.POINTER(SpecBatch), C.c_void_p]),
    "zs_lane_argmax": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint64, C.c_void_p, C.c_void_p]),
    "zs_lane_sample": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint64, C.c_void_p, C.c_void_p,
                                 C.c_void_p, C.c_void_p]),
    "zs_lane_topk": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint64, C.c_uint32, C.c_void_p,
                               C.c_void_p, C.c_void_p]),
    "zs_lane_sample_topk": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p,
                                      C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "zs_step_seed": (C.c_uint32, [C.c_uint32, C.c_uint32]),
    "zs_lane_step": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint64, C.POINTER(LaneStream),
                               C.c_void_p, C.POINTER(C.c_int), C.c_void_p]),
    "zs_last_timings": (C.c_int, [C.c_void_p, C.POINTER(C.c_char_p), C.POINTER(C.c_float), C.c_int]),
    "zs_regex_compile": (C.c_int, [C.c_char_p, C.c_size_t, C.POINTER(C.c_void_p), C.c_char_p, C.c_size_t]),
    "zs_grammar_destroy": (None, [C.c_void_p]),
    "zs_grammar_info": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]),
    "zs_grammar_trans": (C.c_void_p, [C.c_void_p]),
    "zs_grammar_accept": (C.c_void_p, [C.c_void_p]),
    "zs_grammar_dead": (C.c_void_p, [C.c_void_p]),
    "zs_json_schema_regex": (C.c_int, [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t),
                                       C.c_char_p, C.c_size_t]),
    "zs_any_json_regex": (C.c_int, [C.c_uint32, C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t)]),
    "zs_token_table_from_json": (C.c_int, [C.c_char_p, C.c_size_t, C.POINTER(C.c_void_p), C.c_char_p, C.c_size_t]),
    "zs_token_table_from_gguf": (C.c_int, [C.c_char_p, C.POINTER(C.c_void_p), C.c_char_p, C.c_size_t]),
    "zs_token_table_info": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                                      C.POINTER(C.c_int64)]),
    "zs_token_table_offsets": (C.c_void_p, [C.c_void_p]),
    "zs_token_table_bytes": (C.c_void_p, [C.c_void_p]),
    "zs_token_table_valid": (C.c_void_p, [C.c_void_p]),
    "zs_token_table_destroy": (None, [C.c_void_p]),
    "zs_token_table_text": (C.c_int, [C.c_void_p, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)]),
    "zs_hallucination_report": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_float, C.c_float,
                                          C.POINTER(HallucReport)]),
    "zs_hallucination_json": (C.c_int, [C.POINTER(HallucReport), C.c_float, C.c_char_p, C.c_size_t,
                                        C.POINTER(C.c_size_t)]),
    "zs_logprobs_json": (C.c_int, [C.c_int, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p,
                                   C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_char_p, C.c_size_t,
                                   C.POINTER(C.c_size_t)]),
    "zs_tool_call_envelope_regex": (C.c_int, [C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), C.c_uint32, C.c_char_p,
                                              C.c_size_t, C.POINTER(C.c_size_t), C.c_char_p, C.c_size_t]),
}

# ABI version the Structures above describe (include/zs.h ZS_ABI_VERSION)
ABI_VERSION = 2

# zs_struct_layout ids (ZS_LAYOUT_*) of the Structures above
LAYOUTS = {0: Batch, 1: RowParams, 2: SpecBatch, 3: LaneStream, 4: HallucReport}


def layout_mismatches(lib_):
    """Differences between each ctypes Structure and the library's own layout
    of the struct (size and every field offset), as text; empty when equal."""
    out = []
    for which, cls in LAYOUTS.items():
        size = C.c_size_t()
        offs = (C.c_size_t * 64)()
        n = lib_.zs_struct_layout(which, C.byref(size), offs, 64)
        fields = [f[0] for f in cls._fields_]
        if n != len(fields):
            out.append(f"{cls.__name__}: {n} fields in the library, {len(fields)} here")
            continue
        if size.value != C.sizeof(cls):
            out.append(f"{cls.__name__}: size {size.value} != {C.sizeof(cls)}")
        for i, f in enumerate(fields):
            if offs[i] != getattr(cls, f).offset:
                out.append(f"{cls.__name__}.{f}: offset {offs[i]} != {getattr(cls, f).offset}")
    return out


_lib = None


class ZsError(RuntimeError):
    pass


def lib():
    """Load libzs.so (built by zllm_amd.build). Raises if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ZsError(f"{LIB_PATH} not built: run `python -m zllm_amd.build` (hipcc, gfx950)")
        lib_ = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib_, name)
            fn.restype = res
            fn.argtypes = args
        if lib_.zs_abi_version() != ABI_VERSION:
            raise ZsError(f"libzs ABI {lib_.zs_abi_version()} != binding ABI {ABI_VERSION}")
        bad = layout_mismatches(lib_)
        if bad:
            raise ZsError("libzs struct layout differs from the ctypes binding: " + "; ".join(bad))
        _lib = lib_
    return _lib
