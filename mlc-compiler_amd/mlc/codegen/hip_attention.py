"""HIP emitter for :class:`~mlc.kernels.AttentionKernel` (gfx950 MFMA).

Up to 128 keys, every score of a row stays in registers (below); longer rows
use the key-blocked form (``emit_attention_blocked``) with the online-softmax
recurrence. One workgroup of ``W`` waves per (batch-head, block of ``16*W``
queries):

* **staging**: the block's queries, and every key and value of the head,
  are copied from their strided views into LDS with 128-bit loads along
  whichever axis is unit-stride, all loads issued before the first LDS
  store. K is kept as ``[key][d]``, its rows in the order ``mlc::krow``
  gives, and V transposed as ``[d][key]``; row pitches are padded by 8
  elements so the 16-lane phases of ``ds_read_b128`` hit distinct banks.
* **scores**: each wave owns 16 queries and computes ``S^T = K Q^T`` with
  ``v_mfma_f32_16x16x32_f16`` (``_bf16`` for bf16 heads; the body is written
  once over the ``e16``/``v8``/``v4`` aliases) -- A = a 16-key tile of K
  (LDS rows ``16 t .. 16 t + 15``), B = the wave's Q fragment (read once) --
  so lane ``l`` ends up holding query ``l % 16``'s scores for keys
  ``32 (t / 2) + 8 (l / 16) + 4 (t % 2) + i``: eight consecutive keys of
  every 32-key chunk, whose mask words are one 16-byte load. Scores are
  rounded to their storage dtype, as the unfused schedule stores them.
* **row reduction**: the reduction kernel's own steps are rendered per
  element; each query's row lives in four lanes (``l % 16`` fixed), so a
  reduce is a lane-local loop plus two lane exchanges (xor 16 and 32, on
  ``v_permlane16_swap`` / ``v_permlane32_swap``).
* **values**: ``O^T = V^T P^T`` on the same MFMA. The score layout of lane
  ``l`` is exactly the B fragment of ``P^T`` when the 32-element k axis of an
  MFMA is one 32-key chunk (tiles ``2 m`` and ``2 m + 1``), in key order, so
  probabilities never leave registers and a lane's 8 A values are one
  16-byte read of the unpermuted V^T tile. Lane ``l`` ends
  with four consecutive head-dim values of query ``l % 16``: one 8-byte
  store each, at the output's index map over the flat ``[BH, T, D]`` index
  (identity, or the permutation of a folded context copy).

Numerics follow the unfused schedule: fp32 accumulation, scores and
probabilities rounded to their storage dtypes before use, fp32 softmax.
Summation orders differ from the library GEMMs and from the standalone
reduction kernel, and the softmax's exp and division take fast forms
(``FAST_SOFTMAX_MATH``), so results agree to the operands' 16-bit rounding,
not bit for bit.
"""

from __future__ import annotations

import torch

from ..ir.scalar import Call, Ref
from ..kernels import AttentionKernel, Bind
from .hip_backend import (_IDENTITY, _OP, STORAGE, WAVE, LaunchSpec, Renderer, _RowOffsets,
                          _expr_varies, _params, _reciprocal_divisors, _reciprocal_lines,
                          _row_col_access, _scalar_division, axis_terms, bind_defs, cast_code,
                          compute_type, half_inputs, index_type, join_offset, nonpositive_args,
                          render_terms)
from .reduction_schedule import varies_by_column

#: the softmax's exp and its division by the row sum in fast forms
#: (``mlc::exp_fast`` and a multiply by the row reciprocal), and floating-point
#: contraction inside the attention kernels (a scale and a mask add become one
#: mixed-precision FMA on the 16-bit operands). All of it is used only here,
#: where every probability is rounded to fp16 or bf16 before it is used: the
#: errors (about 1e-6, 1.5 fp32 ulp, one fp32 rounding) are far below that
#: rounding.
FAST_SOFTMAX_MATH = True

#: waves per workgroup (each owns 16 queries): ``waves`` forces a count;
#: otherwise the largest of ``choices`` that still gives ``min_workgroups``
#: workgroups (one per CU), else the smallest. Measured on MI355X for BERT's
#: 128 x 128 x 64 heads: 12 heads -> 2 waves (5.3 us vs 5.7 at 4 and 7.0 at
#: 8); 384 heads -> 8 waves (12.6 us vs 14.8 at 4, 18.3 at 2).
ATTENTION_TUNING = {"waves": None, "choices": (8, 4, 2), "min_workgroups": 256}

#: halfs of padding after each LDS row of Q, K and V^T (a multiple of 8, so
#: every row starts 16-byte aligned for the 128-bit operand reads)
LDS_ROW_PAD = 8


def attention_waves(heads: int, queries: int) -> int:
    forced = ATTENTION_TUNING["waves"]
    if forced:
        return max(1, min(forced, queries // 16))
    choices = [w for w in ATTENTION_TUNING["choices"] if 16 * w <= max(16, queries)] or [1]
    for w in choices:
        if heads * -(-queries // (16 * w)) >= ATTENTION_TUNING["min_workgroups"]:
            return w
    return choices[-1]


class _FastExpRenderer(Renderer):
    """``exp`` as ``mlc::exp_fast``; ``exp(x - rowmax(x))`` as
    ``mlc::exp_fast_shift`` (one fma forms ``x log2 e - RN(m log2 e)``: the
    rounding of ``m log2 e`` for the row's maximum ``m`` is the same factor on
    every exp of the row and cancels in the normalisation). ``nonpos`` holds
    the ``x - rowmax(x)`` expressions (``nonpositive_args``); the exp of any
    other difference keeps its own rounding and is ``exp_fast`` of it."""

    def __init__(self, operand, temp, half_slots=frozenset(), defs=None, nonpos=frozenset()):
        super().__init__(operand, temp, half_slots, defs)
        self.nonpos = nonpos

    def _call(self, e):
        if e.fn == "exp":
            x = e.args[0]
            shift = x in self.nonpos
            if isinstance(x, Ref) and isinstance(self.defs.get(x.name), Call):
                x = self.defs[x.name]  # a bind holding the difference
            if shift and isinstance(x, Call) and x.fn == "sub":
                (a, ta), (b, tb) = self(x.args[0]), self(x.args[1])
                if ta == "float" and tb == "float":
                    return f"mlc::exp_fast_shift({a}, {b})", "float"
            code, t = self(x)
            if t == "float":
                return f"mlc::exp_fast({code})", "float"
        return super()._call(e)


#: 16-bit element, 8- and 4-element vector types of the operands, per dtype
_TYPES = {torch.float16: ("mlc::f16", "mlc::half8", "mlc::half4"),
          torch.bfloat16: ("__bf16", "mlc::bf16x8", "mlc::bf16x4")}


def _type_aliases(k: AttentionKernel) -> str:
    """The kernel body is written over ``e16``/``v8``/``v4``; these bind them
    to the operands' 16-bit float type (conversions to ``e16`` round to
    nearest even, as the unfused schedule's stores do)."""
    e, v8, v4 = _TYPES[k.q.dtype]
    return f"  using e16 = {e};\n  using v8 = {v8};\n  using v4 = {v4};"


def _stage(tag: str, lds: str, src: str, base: str, R: int, C: int, sr: int, sc: int, pr: int,
           pc: int, aligned_c: bool, aligned_r: bool, threads: int, rows_valid: str | None,
           it: str, key_rows: bool = False) -> tuple[list[str], list[str]]:
    """Copy the R x C tile ``src[base + r*sr + c*sc]`` to ``lds[r*pr + c*pc]``
    (``lds[krow(r)*pr + c*pc]`` with ``key_rows``, for the K tile: the key
    order the score MFMAs read, ``mlc::krow``).

    Returns (load lines, store lines): every load of every operand is issued
    before the first LDS store, so the workgroup waits for memory once, not
    once per loop trip."""
    rr = "mlc::krow(r)" if key_rows else "r"
    load: list[str] = []
    store: list[str] = []
    if sc == 1 and C % 8 == 0 and aligned_c:
        mode, per = "c", 8
    elif sr == 1 and R % 8 == 0 and aligned_r and not rows_valid:
        mode, per = "r", 8
    else:
        mode, per = "s", 1
    n = R * C // per
    trips = -(-n // threads)
    full = n % threads == 0
    ty = "v8" if per == 8 else "e16"
    load.append(f"  {ty} {tag}[{trips}];")
    load.append("#pragma unroll")
    load.append(f"  for (int u = 0; u < {trips}; ++u) {{")
    load.append(f"    const int e = (int)threadIdx.x + u * {threads};")
    store.append("#pragma unroll")
    store.append(f"  for (int u = 0; u < {trips}; ++u) {{")
    store.append(f"    const int e = (int)threadIdx.x + u * {threads};")
    conds = [] if full else [f"e < {n}"]
    if mode == "c":
        rc = f"const int r = e / {C // 8}, c = (e % {C // 8}) * 8;"
        addr = f"{src} + {base} + ({it})r * ({it}){sr} + ({it})c"
    elif mode == "r":
        rc = f"const int c = e / {R // 8}, r = (e % {R // 8}) * 8;"
        addr = f"{src} + {base} + ({it})r + ({it})c * ({it}){sc}"
    else:
        rc = f"const int r = e / {C}, c = e % {C};"
        addr = None
    if rows_valid:
        conds.append(f"r < {rows_valid}")
    guard = f"if ({' && '.join(conds)}) " if conds else ""
    load.append(f"    {rc}")
    store.append(f"    {rc}")
    if per == 8:
        load.append(f"    {guard}{tag}[u] = *reinterpret_cast<const v8*>({addr});")
        if mode == "c" and pc == 1 and pr % 8 == 0:
            store.append(f"    {guard}*reinterpret_cast<v8*>({lds} + {rr} * {pr} + c) = {tag}[u];")
        elif mode == "r" and pr == 1 and pc % 8 == 0 and not key_rows:
            store.append(f"    {guard}*reinterpret_cast<v8*>({lds} + r + c * {pc}) = {tag}[u];")
        else:
            if mode == "c":  # one row, 8 columns
                row, col = rr, "(c + j)"
            else:  # 8 rows, one column
                row, col = ("mlc::krow(r + j)" if key_rows else "(r + j)"), "c"
            store.append(f"    {guard}{{")
            store.append("#pragma unroll")
            store.append(f"      for (int j = 0; j < 8; ++j) {lds}[{row} * {pr} + {col} * {pc}] "
                         f"= {tag}[u][j];")
            store.append("    }")
    else:
        load.append(f"    {guard}{tag}[u] = *reinterpret_cast<const e16*>({src} + {base} + ({it})r * ({it}){sr} + ({it})c * ({it}){sc});")
        store.append(f"    {guard}{lds}[{rr} * {pr} + c * {pc}] = {tag}[u];")
    load.append("  }")
    store.append("  }")
    return load, store


#: XCDs of one MI355X; workgroups are dispatched to them round-robin by index
XCDS = 8


def _tile_of_workgroup(BH: int, NQB: int, QB: int, it: str) -> list[str]:
    """``bh`` and ``q0`` of this workgroup. Workgroup ``i`` runs on XCD
    ``i % 8``, and every XCD has its own L2. When a head has several query
    tiles and the heads divide evenly over the XCDs, a head's tiles are given
    to workgroups on one XCD, so its keys and values are fetched into one L2
    once rather than into several."""
    if NQB > 1 and BH % XCDS == 0:
        return [f"  const uint32_t xcd = blockIdx.x % {XCDS}, slot = blockIdx.x / {XCDS};",
                f"  const {it} bh = ({it})((slot / {NQB}) * {XCDS} + xcd);",
                f"  const int q0 = (int)(slot % {NQB}) * {QB};"]
    if NQB > 1 and (BH * NQB) % XCDS == 0:
        # XCD x takes a contiguous run of the (head, tile) list: a head's tiles
        # span at most two XCDs
        per = BH * NQB // XCDS
        return [f"  const uint32_t item = (blockIdx.x % {XCDS}) * {per} + blockIdx.x / {XCDS};",
                f"  const {it} bh = ({it})(item / {NQB});",
                f"  const int q0 = (int)(item % {NQB}) * {QB};"]
    return [f"  const {it} bh = ({it})(blockIdx.x / {NQB});",
            f"  const int q0 = (int)(blockIdx.x % {NQB}) * {QB};"]


def _round_scores(acc: str, dst: str, dtype: torch.dtype, ind: str) -> list[str]:
    """A score tile's four fp32 accumulators rounded to the scores' storage
    dtype, as the unfused schedule stores them. fp16 rounds the four in two
    packed conversions; the fp32 copies read back are what the softmax's
    mixed-precision fmas take in as fp16 operands. (Pairs, not the four at
    once: a pair converts with one v_cvt_pk_f16_f32.)"""
    if dtype == torch.float16:
        return [f"{ind}{{ const mlc::half2v h0 = __builtin_convertvector("
                f"(mlc::float2v){{{acc}[0], {acc}[1]}}, mlc::half2v);",
                f"{ind}  const mlc::half2v h1 = __builtin_convertvector("
                f"(mlc::float2v){{{acc}[2], {acc}[3]}}, mlc::half2v);",
                f"{ind}  {dst}[0] = (float)h0[0]; {dst}[1] = (float)h0[1];",
                f"{ind}  {dst}[2] = (float)h1[0]; {dst}[3] = (float)h1[1]; }}"]
    return ["#pragma unroll",
            f"{ind}for (int i = 0; i < 4; ++i) {dst}[i] = {cast_code(acc + '[i]', dtype)[0]};"]


def _lane_words(sm, a, dst: str, base: str, c0: str, offs, it: str, ind: str) -> list[str]:
    """The 8 words of column operand ``a`` at keys ``c0 .. c0 + 7`` into
    ``dst[0..7]``: one 16-byte load when the row's columns are unit-stride
    and 16-byte aligned, two 8-byte loads at 8-byte alignment, else one load
    per word. ``c0`` is a multiple of 8 (a lane's keys, ``mlc::krow``)."""
    S = STORAGE[a.dtype]
    out = [f"{ind}{{ const {it} c0 = ({it})({c0});"]
    for V in (8, 4):
        acc = _row_col_access(sm, a, V)
        if acc.mode == "affine" and acc.aligned:
            out.append("#pragma unroll")
            out.append(f"{ind}  for (int h = 0; h < {8 // V}; ++h) {{")
            out.append(f"{ind}    const mlc::pack<{S}, {V}> w_ = *reinterpret_cast<const mlc::pack<{S}, {V}>*>"
                       f"({base} + {offs.col(a, f'(c0 + ({it})(h * {V}))')});")
            out.append("#pragma unroll")
            out.append(f"{ind}    for (int j = 0; j < {V}; ++j) {dst}[h * {V} + j] = w_.x[j];")
            out.append(f"{ind}  }}")
            break
    else:
        out.append("#pragma unroll")
        out.append(f"{ind}  for (int j = 0; j < 8; ++j) {dst}[j] = "
                   f"({base})[{offs.col(a, f'(c0 + ({it})j)')}];")
    out.append(f"{ind}}}")
    return out


def _aligned(offset: int, strides) -> bool:
    return offset % 8 == 0 and all(s % 8 == 0 for s in strides)


#: the most keys whose scores one wave holds in registers (the single-pass form)
MAX_RESIDENT_KEYS = 128


def emit_attention(k: AttentionKernel, cfg=None) -> tuple[str, LaunchSpec]:
    if k.kt.shape[2] > MAX_RESIDENT_KEYS:
        return emit_attention_blocked(k, cfg)
    sm = k.softmax
    BH, T, D = k.q.shape
    Tk = k.kt.shape[2]
    NT = Tk // 16
    W = attention_waves(BH, T)
    QB = 16 * W
    NQB = -(-T // QB)
    THREADS = W * WAVE
    it = index_type(k)
    PK, PV, PQ = D + LDS_ROW_PAD, Tk + LDS_ROW_PAD, D + LDS_ROW_PAD
    lds_bytes = 2 * (Tk * PK + D * PV + QB * PQ)

    L: list[str] = []
    L.append(f"extern \"C\" __global__ void __launch_bounds__({THREADS}) "
             f"KERNEL({', '.join(_params(k))}) {{")
    L.append(f"  // attention: {BH} heads x [{T} x {D}] x [{Tk}]; {QB} queries per workgroup, "
             f"16 per wave")
    if FAST_SOFTMAX_MATH:
        L.append("#pragma clang fp contract(fast)")
    L.append(_type_aliases(k))
    L.append(f"  __shared__ __align__(16) e16 ks[{Tk * PK}];")
    L.append(f"  __shared__ __align__(16) e16 vt[{D * PV}];")
    L.append(f"  __shared__ __align__(16) e16 qs[{QB * PQ}];")
    L += _tile_of_workgroup(BH, NQB, QB, it)

    ql_ = k.q.layout
    qsb, qsr, qsc = ql_.strides
    rows_valid = None
    if T % QB:
        L.append(f"  const int qn = {T} - q0 < {QB} ? {T} - q0 : {QB};")
        rows_valid = "qn"
    q_ld, q_st = _stage("gq", "qs", "in0",
                        f"(({it}){ql_.offset} + bh * ({it}){qsb} + ({it})q0 * ({it}){qsr})",
                        QB, D, qsr, qsc, PQ, 1, _aligned(ql_.offset, (qsb, qsr)),
                        _aligned(ql_.offset, (qsb, qsc)), THREADS, rows_valid, it)
    # kt is [BH, D, Tk]: key r, dim c sits at r*sk + c*sd
    kl = k.kt.layout
    ksb, ksd, ksk = kl.strides
    k_ld, k_st = _stage("gk", "ks", "in1", f"(({it}){kl.offset} + bh * ({it}){ksb})", Tk, D, ksk,
                        ksd, PK, 1, _aligned(kl.offset, (ksb, ksk)),
                        _aligned(kl.offset, (ksb, ksd)), THREADS, None, it, key_rows=True)
    # v is [BH, Tk, D], staged transposed as [d][key]
    vl = k.v.layout
    vsb, vsk, vsd = vl.strides
    v_ld, v_st = _stage("gv", "vt", "in2", f"(({it}){vl.offset} + bh * ({it}){vsb})", Tk, D, vsk,
                        vsd, 1, PV, _aligned(vl.offset, (vsb, vsk)),
                        _aligned(vl.offset, (vsb, vsd)), THREADS, None, it)
    L += q_ld + k_ld + v_ld + q_st + k_st + v_st
    L.append("  __syncthreads();")
    L.append("  const int w = threadIdx.x / 64, l = threadIdx.x % 64;")
    L.append("  const int ql = l % 16, g = l / 16;")
    L.append("  const int qw = q0 + w * 16;")
    L.append(f"  if (qw >= {T}) return;  // no barrier follows")
    # scores
    L.append(f"  v8 qf[{D // 32}];")
    L.append("#pragma unroll")
    L.append(f"  for (int dc = 0; dc < {D // 32}; ++dc)")
    L.append(f"    qf[dc] = *reinterpret_cast<const v8*>(qs + (w * 16 + ql) * {PQ} + dc * 32 + g * 8);")
    L.append(f"  float s[{NT}][4];")
    L.append("#pragma unroll")
    L.append(f"  for (int t = 0; t < {NT}; ++t) {{")
    L.append("    mlc::float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};")
    L.append("#pragma unroll")
    L.append(f"    for (int dc = 0; dc < {D // 32}; ++dc) {{")
    L.append(f"      const v8 kf = *reinterpret_cast<const v8*>(ks + (t * 16 + ql) * {PK} + dc * 32 + g * 8);")
    L.append("      acc = mlc::mfma_16x16x32(kf, qf[dc], acc);")
    L.append("    }")
    L += _round_scores("acc", "s[t]", k.score_dtype, "    ")
    L.append("  }")
    L.append(f"  const {it} row = bh * ({it}){T} + ({it})(qw + ql);")

    # the reduction's other operands
    offs = _RowOffsets(sm, it)
    vector = varies_by_column(sm)
    col_slots = [i for i, a in enumerate(sm.inputs) if a.index.varies_along("col")]
    param = {}
    n = 3
    for i in range(len(sm.inputs)):
        if i != k.score_slot:
            param[i] = n
            n += 1
    in_types = {i: compute_type(a.dtype) for i, a in enumerate(sm.inputs)}
    for i, a in enumerate(sm.inputs):
        if i == k.score_slot:
            continue
        p, ct = param[i], in_types[i]
        if i not in col_slots:
            L.append(f"  const {ct} x{i} = mlc::ld(in{p} + {offs.row(a)});")
            continue
        L.append(f"  {ct} x{i}[{NT}][4];")
        L.append(f"  {{ const {it} rb = {offs.row(a)};")
        L.append("#pragma unroll")
        L.append(f"    for (int m = 0; m < {NT // 2}; ++m) {{")
        L.append(f"      {STORAGE[a.dtype]} w[8];")
        L += _lane_words(sm, a, "w", f"in{p} + rb", "m * 32 + g * 8", offs, it, "      ")
        L.append("#pragma unroll")
        L.append("      for (int j = 0; j < 4; ++j) {")
        L.append(f"        x{i}[2 * m][j] = mlc::ld(&w[j]);")
        L.append(f"        x{i}[2 * m + 1][j] = mlc::ld(&w[4 + j]);")
        L.append("      }")
        L.append("    }")
        L.append("  }")

    temp_types: dict[str, str] = {}

    def ref_elem(slot):
        if slot == k.score_slot:
            return "s[t][i]", "float"
        if slot in col_slots:
            return f"x{slot}[t][i]", in_types[slot]
        return f"x{slot}", in_types[slot]

    def ref_scalar(slot):
        if slot == k.score_slot or slot in col_slots:
            raise AssertionError("column operand read in a row-scalar expression")
        return f"x{slot}", in_types[slot]

    def temp_elem(name):
        return (f"{name}[t][i]" if name in vector else name), temp_types[name]

    def temp_scalar(name):
        if name in vector:
            raise AssertionError("vector temp read in a row-scalar expression")
        return name, temp_types[name]

    half, defs = half_inputs(sm), bind_defs(sm)
    if FAST_SOFTMAX_MATH:
        nonpos = frozenset(nonpositive_args(sm))
        elem_r = _FastExpRenderer(ref_elem, temp_elem, half, defs, nonpos)
        scal_r = _FastExpRenderer(ref_scalar, temp_scalar, half, defs, nonpos)
    else:
        elem_r, scal_r = Renderer(ref_elem, temp_elem, half, defs), Renderer(ref_scalar, temp_scalar, half, defs)
    rcp_for = _reciprocal_divisors(sm, vector)
    score_cols = set(col_slots) | {k.score_slot}

    def elem_loop(target: str, code: str) -> list[str]:
        return ["#pragma unroll", f"  for (int t = 0; t < {NT}; ++t)", "#pragma unroll",
                "    for (int i = 0; i < 4; ++i)", f"      {target}[t][i] = {code};"]

    for st in sm.steps:
        if isinstance(st, Bind):
            if st.name in vector:
                code, t = elem_r(st.expr)
                temp_types[st.name] = t
                L.append(f"  {t} {st.name}[{NT}][4];")
                sd = _scalar_division(st.expr, rcp_for)
                if sd is not None and t == "float":
                    num, d = elem_r(sd[0])[0], sd[1]
                    L.append(f"  if (__all(ok_{d})) {{")
                    fast = (f"({num} * rcp_{d})" if FAST_SOFTMAX_MATH
                            else f"mlc::div_rcp({num}, {d}, rcp_{d})")
                    L += elem_loop(st.name, fast)
                    L.append("  } else {")
                    L += elem_loop(st.name, code)
                    L.append("  }")
                else:
                    L += elem_loop(st.name, code)
            else:
                code, t = scal_r(st.expr)
                temp_types[st.name] = t
                L.append(f"  const {t} {st.name} = {code};")
                L += _reciprocal_lines(st.name, rcp_for)
            continue
        code, t = elem_r(st.expr) if _expr_varies(st.expr, score_cols, vector) else scal_r(st.expr)
        if t == "bool":
            code, t = f"((int64_t)({code}))", "int64_t"
        temp_types[st.name] = t
        op = _OP[st.kind]
        L.append(f"  {t} {st.name};")
        L.append("  {")
        L.append(f"    {t} acc = {_IDENTITY[st.kind][t]};")
        L.append("#pragma unroll")
        L.append(f"    for (int t = 0; t < {NT}; ++t)")
        L.append("#pragma unroll")
        L.append(f"      for (int i = 0; i < 4; ++i) acc = {op}::f(acc, ({t})({code}));")
        if t == "float":
            L.append(f"    acc = mlc::xor32<{op}>(mlc::xor16<{op}>(acc));")
        else:
            L.append(f"    acc = {op}::f(acc, __shfl_xor(acc, 16, 64));")
            L.append(f"    acc = {op}::f(acc, __shfl_xor(acc, 32, 64));")
        L.append(f"    {st.name} = acc;")
        L.append("  }")
        L += _reciprocal_lines(st.name, rcp_for)

    # probabilities, rounded to their storage dtype
    prob = sm.outputs[0].value
    e = sm.out_expr[prob.name]
    code, _ = elem_r(e) if _expr_varies(e, score_cols, vector) else scal_r(e)
    L.append(f"  float pr[{NT}][4];")
    L += elem_loop("pr", cast_code(code, k.prob_dtype)[0])
    # O^T = V^T P^T, two 16-key tiles per MFMA
    L.append("#pragma unroll")
    L.append(f"  for (int dt = 0; dt < {D // 16}; ++dt) {{")
    L.append("    mlc::float4v o = {0.0f, 0.0f, 0.0f, 0.0f};")
    L.append(f"    const e16* vrow = vt + (dt * 16 + ql) * {PV} + g * 8;")
    L.append("#pragma unroll")
    L.append(f"    for (int m = 0; m < {NT // 2}; ++m) {{")
    L.append("      const v8 a = *reinterpret_cast<const v8*>(vrow + m * 32);")
    L.append("      const v8 b = {(e16)pr[2 * m][0], (e16)pr[2 * m][1], "
             "(e16)pr[2 * m][2], (e16)pr[2 * m][3], (e16)pr[2 * m + 1][0], "
             "(e16)pr[2 * m + 1][1], (e16)pr[2 * m + 1][2], (e16)pr[2 * m + 1][3]};")
    L.append("      o = mlc::mfma_16x16x32(a, b, o);")
    L.append("    }")
    omap = k.outputs[0].index
    parts = render_terms(axis_terms(omap, "idx"), BH * T * D, "f0", it)
    if omap.base:
        parts.append(f"({it}){omap.base}")
    L.append(f"    const v4 h = {{(e16)o[0], (e16)o[1], (e16)o[2], (e16)o[3]}};")
    L.append(f"    const {it} f0 = row * ({it}){D} + ({it})(dt * 16 + g * 4);")
    L.append(f"    *reinterpret_cast<v4*>(out0 + {join_offset(parts, it)}) = h;")
    L.append("  }")
    L.append("}")
    spec = LaunchSpec("", BH * NQB, THREADS, lds_bytes,
                      {"kind": "attention", "heads": BH, "queries": T, "keys": Tk, "head_dim": D,
                       "queries_per_wg": QB})
    return "\n".join(L), spec



# --------------------------------------------------------------------------
# key-blocked form (more keys than one workgroup holds)
# --------------------------------------------------------------------------

#: keys per block of the blocked kernel
KEY_BLOCK = 64


def blocked_form(sm):
    """The online-softmax structure of ``sm`` when it is exactly
    ``cast?(exp(x - max(x)) / sum(exp(x - max(x))))`` over its row, else None.
    The blocked kernel needs it: it keeps a running max and sum per row and
    rescales its partial output, instead of holding the whole row."""
    from ..ir.scalar import Call, Cast, Ref
    from .reduction_schedule import detect_online_softmax

    online = detect_online_softmax(sm)
    if online is None or len(sm.outputs) != 1 or sm.row_outputs:
        return None
    by_name = {s.name: s for s in sm.steps}

    def through(e):
        while True:
            if isinstance(e, Ref) and isinstance(by_name.get(e.name), Bind):
                e = by_name[e.name].expr
            elif isinstance(e, Cast):
                e = e.x
            else:
                return e

    out = through(sm.out_expr[sm.outputs[0].value.name])
    if not (isinstance(out, Call) and out.fn == "div" and isinstance(out.args[1], Ref)
            and out.args[1].name == online.sum_step.name):
        return None
    if through(out.args[0]) != through(online.sum_step.expr):
        return None
    return online


def emit_attention_blocked(k: AttentionKernel, cfg=None) -> tuple[str, LaunchSpec]:
    """Key-blocked attention: each workgroup streams the head's keys and
    values through LDS in blocks of ``KEY_BLOCK``, keeping per query row a
    running max ``m`` and sum ``l`` (the online-softmax recurrence) and an
    fp32 output accumulator rescaled by ``exp(m_old - m_new)`` per block; the
    division by ``l`` happens once at the end. The next block's loads are in
    flight while the current block computes."""
    from .reduction_schedule import dependencies

    sm = k.softmax
    online = blocked_form(sm)
    assert online is not None, "not an online-softmax reduction"
    BH, T, D = k.q.shape
    Tk = k.kt.shape[2]
    KB = KEY_BLOCK
    NB = Tk // KB
    NT = KB // 16
    W = attention_waves(BH, T)
    QB = 16 * W
    NQB = -(-T // QB)
    THREADS = W * WAVE
    it = index_type(k)
    PK, PV, PQ = D + LDS_ROW_PAD, KB + LDS_ROW_PAD, D + LDS_ROW_PAD
    lds_bytes = 2 * (KB * PK + D * PV + QB * PQ)

    L: list[str] = []
    L.append(f"extern \"C\" __global__ void __launch_bounds__({THREADS}) "
             f"KERNEL({', '.join(_params(k))}) {{")
    L.append(f"  // attention, key-blocked: {BH} heads x [{T} x {D}] x [{Tk}] in {NB} blocks of "
             f"{KB} keys; {QB} queries per workgroup, 16 per wave; online softmax")
    if FAST_SOFTMAX_MATH:
        L.append("#pragma clang fp contract(fast)")
    L.append(_type_aliases(k))
    L.append(f"  __shared__ __align__(16) e16 ks[{KB * PK}];")
    L.append(f"  __shared__ __align__(16) e16 vt[{D * PV}];")
    L.append(f"  __shared__ __align__(16) e16 qs[{QB * PQ}];")
    L += _tile_of_workgroup(BH, NQB, QB, it)
    ql_ = k.q.layout
    qsb, qsr, qsc = ql_.strides
    # query tile j of a head holds the half-tiles j and 2 NQB - 1 - j (waves
    # 0 .. W/2 - 1 and W/2 .. W - 1): under a causal mask every workgroup then
    # has the same number of unmasked keys, so no late, long workgroup sets
    # the kernel's end; any other mask is indifferent to the pairing
    fold = T % QB == 0 and W % 2 == 0 and NQB > 1
    if fold:
        H = QB // 2
        L.append(f"  const int qa = (q0 / {QB}) * {H}, qb = ({2 * NQB - 1} - q0 / {QB}) * {H};")
        q_ld, q_st = [], []
        for tag, lds, first in (("gq", "qs", "qa"), ("gq2", f"(qs + {H * PQ})", "qb")):
            ld_, st_ = _stage(tag, lds, "in0",
                              f"(({it}){ql_.offset} + bh * ({it}){qsb} + ({it}){first} * ({it}){qsr})",
                              H, D, qsr, qsc, PQ, 1, _aligned(ql_.offset, (qsb, qsr)),
                              _aligned(ql_.offset, (qsb, qsc)), THREADS, None, it)
            q_ld += ld_
            q_st += st_
    else:
        rows_valid = None
        if T % QB:
            L.append(f"  const int qn = {T} - q0 < {QB} ? {T} - q0 : {QB};")
            rows_valid = "qn"
        q_ld, q_st = _stage("gq", "qs", "in0",
                            f"(({it}){ql_.offset} + bh * ({it}){qsb} + ({it})q0 * ({it}){qsr})",
                            QB, D, qsr, qsc, PQ, 1, _aligned(ql_.offset, (qsb, qsr)),
                            _aligned(ql_.offset, (qsb, qsc)), THREADS, rows_valid, it)
    kl = k.kt.layout
    ksb, ksd, ksk = kl.strides
    k_ld, k_st = _stage("gk", "ks", "in1",
                        f"(({it}){kl.offset} + bh * ({it}){ksb} + ({it})kb0 * ({it}){ksk})",
                        KB, D, ksk, ksd, PK, 1, _aligned(kl.offset, (ksb, ksk, KB * ksk)),
                        _aligned(kl.offset, (ksb, ksd, KB * ksk)), THREADS, None, it,
                        key_rows=True)
    vl = k.v.layout
    vsb, vsk, vsd = vl.strides
    v_ld, v_st = _stage("gv", "vt", "in2",
                        f"(({it}){vl.offset} + bh * ({it}){vsb} + ({it})kb0 * ({it}){vsk})",
                        KB, D, vsk, vsd, 1, PV, _aligned(vl.offset, (vsb, vsk, KB * vsk)),
                        _aligned(vl.offset, (vsb, vsd, KB * vsk)), THREADS, None, it)
    # declarations hoisted out of the block loop
    L += q_ld + q_st
    L += [k_ld[0], v_ld[0]]
    L.append("  int kb0 = 0;")
    L += k_ld[1:] + v_ld[1:] + k_st + v_st
    L.append("  __syncthreads();")
    L.append("  const int w = threadIdx.x / 64, l = threadIdx.x % 64;")
    L.append("  const int ql = l % 16, g = l / 16;")
    if fold:
        L.append(f"  const int qw = w < {W // 2} ? qa + w * 16 : qb + (w - {W // 2}) * 16;")
    else:
        L.append("  const int qw = q0 + w * 16;")
    L.append(f"  const bool active = qw < {T};  // wave-uniform; every wave meets every barrier")
    L.append(f"  const {it} row = bh * ({it}){T} + ({it})(active ? qw + ql : 0);")
    L.append(f"  v8 qf[{D // 32}];")
    L.append("#pragma unroll")
    L.append(f"  for (int dc = 0; dc < {D // 32}; ++dc)")
    L.append(f"    qf[dc] = *reinterpret_cast<const v8*>(qs + (w * 16 + ql) * {PQ} + dc * 32 + g * 8);")
    L.append("  float m_run = (-__builtin_huge_valf()), l_run = 0.0f;")
    if FAST_SOFTMAX_MATH:
        L.append("  float ml_run = (-__builtin_huge_valf());  // RN(m_run log2 e)")
    L.append(f"  mlc::float4v o[{D // 16}];")
    L.append("#pragma unroll")
    L.append(f"  for (int dt = 0; dt < {D // 16}; ++dt) o[dt] = mlc::float4v{{0.0f, 0.0f, 0.0f, 0.0f}};")

    # the reduction's operands other than the scores; row-constant ones once
    offs = _RowOffsets(sm, it)
    vector = varies_by_column(sm)
    col_slots = [i for i, a in enumerate(sm.inputs) if a.index.varies_along("col")]
    param = {}
    n = 3
    for i in range(len(sm.inputs)):
        if i != k.score_slot:
            param[i] = n
            n += 1
    in_types = {i: compute_type(a.dtype) for i, a in enumerate(sm.inputs)}
    for i, a in enumerate(sm.inputs):
        if i != k.score_slot and i not in col_slots:
            L.append(f"  const {in_types[i]} x{i} = mlc::ld(in{param[i]} + {offs.row(a)});")
    temp_types: dict[str, str] = {}

    def ref_elem(slot):
        if slot == k.score_slot:
            return "s[t][i]", "float"
        if slot in col_slots:
            return f"x{slot}[t][i]", in_types[slot]
        return f"x{slot}", in_types[slot]

    def ref_scalar(slot):
        if slot == k.score_slot or slot in col_slots:
            raise AssertionError("column operand read in a row-scalar expression")
        return f"x{slot}", in_types[slot]

    def temp_elem(name):
        return (f"{name}[t][i]" if name in vector else name), temp_types[name]

    def temp_scalar(name):
        if name in vector:
            raise AssertionError("vector temp read in a row-scalar expression")
        return name, temp_types[name]

    half, defs = half_inputs(sm), bind_defs(sm)
    if FAST_SOFTMAX_MATH:
        nonpos = frozenset(nonpositive_args(sm))
        elem_r = _FastExpRenderer(ref_elem, temp_elem, half, defs, nonpos)
        scal_r = _FastExpRenderer(ref_scalar, temp_scalar, half, defs, nonpos)
    else:
        elem_r, scal_r = Renderer(ref_elem, temp_elem, half, defs), Renderer(ref_scalar, temp_scalar, half, defs)
    deps = dependencies(sm.steps)
    needed = deps[online.max_step.name]
    by_name = {s.name: s for s in sm.steps}
    # row-constant binds the maxed value needs, before the loop
    for nm in [s.name for s in sm.steps if s.name in needed]:
        st = by_name[nm]
        if isinstance(st, Bind) and nm not in vector:
            code, t = scal_r(st.expr)
            temp_types[nm] = t
            L.append(f"  const {t} {nm} = {code};")
    exp_ = "mlc::exp_fast" if FAST_SOFTMAX_MATH else "mlc::exp_"

    mask_slots = [i for i in col_slots if i != k.score_slot]

    def mask_loads(kc: str, ind: str) -> list[str]:
        out = []
        for i in mask_slots:
            a = sm.inputs[i]
            out.append(f"{ind}{{ const {it} rb = {offs.row(a)};")
            out.append("#pragma unroll")
            out.append(f"{ind}  for (int m = 0; m < {NT // 2}; ++m) {{")
            out += _lane_words(sm, a, f"xr{i}[m].x", f"in{param[i]} + rb",
                               f"{kc} + m * 32 + g * 8", offs, it, ind + "    ")
            out.append(f"{ind}  }}")
            out.append(f"{ind}}}")
        return out

    for i in mask_slots:
        L.append(f"  mlc::pack<{STORAGE[sm.inputs[i].dtype]}, 8> xr{i}[{NT // 2}];")
    if mask_slots:
        L.append("  if (active) {")
        L += mask_loads("0", "    ")
        L.append("  }")

    L.append(f"  for (int b = 0; b < {NB}; ++b) {{")
    L.append(f"    if (b + 1 < {NB}) {{  // next block's loads, in flight during this block's math")
    L.append(f"      kb0 = (b + 1) * {KB};")
    L += ["    " + x for x in k_ld[1:] + v_ld[1:]]
    L.append("    }")
    L.append("    if (active) {")
    L.append(f"      const int kc = b * {KB};")
    # every tile's operands of one head-dim chunk are read before its MFMAs,
    # and the tiles' four accumulations are independent: LDS and MFMA latency
    # overlap instead of alternating (each tile still sums its chunks in order)
    L.append(f"      mlc::float4v acc[{NT}];")
    L.append("#pragma unroll")
    L.append(f"      for (int t = 0; t < {NT}; ++t) acc[t] = mlc::float4v{{0.0f, 0.0f, 0.0f, 0.0f}};")
    L.append("#pragma unroll")
    L.append(f"      for (int dc = 0; dc < {D // 32}; ++dc) {{")
    L.append(f"        v8 kf[{NT}];")
    L.append("#pragma unroll")
    L.append(f"        for (int t = 0; t < {NT}; ++t) kf[t] = *reinterpret_cast<const v8*>(ks + (t * 16 + ql) * {PK} + dc * 32 + g * 8);")
    L.append("#pragma unroll")
    L.append(f"        for (int t = 0; t < {NT}; ++t) acc[t] = mlc::mfma_16x16x32(kf[t], qf[dc], acc[t]);")
    L.append("      }")
    L.append(f"      float s[{NT}][4];")
    L.append("#pragma unroll")
    L.append(f"      for (int t = 0; t < {NT}; ++t) {{")
    L += _round_scores("acc[t]", "s[t]", k.score_dtype, "        ")
    L.append("      }")
    # the other column operands (the mask): widened from the words loaded one
    # block ahead, then the next block's words are requested, so their memory
    # latency overlaps this block's work as the K/V tiles' does
    for i in mask_slots:
        L.append(f"      {in_types[i]} x{i}[{NT}][4];")
        L.append("#pragma unroll")
        L.append(f"      for (int t = 0; t < {NT}; ++t)")
        L.append("#pragma unroll")
        L.append(f"        for (int j = 0; j < 4; ++j) x{i}[t][j] = mlc::ld(&xr{i}[t / 2].x[(t % 2) * 4 + j]);")
    if mask_slots:
        L.append(f"      if (b + 1 < {NB}) {{")
        L += mask_loads("(kc + " + str(KB) + ")", "        ")
        L.append("      }")
    for nm in [s.name for s in sm.steps if s.name in needed]:
        st = by_name[nm]
        if isinstance(st, Bind) and nm in vector:
            code, t = elem_r(st.expr)
            temp_types[nm] = t
            L.append(f"      {t} {nm}[{NT}][4];")
            L.append("#pragma unroll")
            L.append(f"      for (int t = 0; t < {NT}; ++t)")
            L.append("#pragma unroll")
            L.append(f"        for (int i = 0; i < 4; ++i) {nm}[t][i] = {code};")
    xcode, _ = elem_r(online.value)
    L.append(f"      float x[{NT}][4];")
    L.append("      float mb = (-__builtin_huge_valf());")
    L.append("#pragma unroll")
    L.append(f"      for (int t = 0; t < {NT}; ++t)")
    L.append("#pragma unroll")
    L.append("        for (int i = 0; i < 4; ++i) {")
    L.append(f"          x[t][i] = (float)({xcode});")
    L.append("          mb = mlc::max_<float>(mb, x[t][i]);")
    L.append("        }")
    L.append("      mb = mlc::xor32<mlc::OpMax>(mlc::xor16<mlc::OpMax>(mb));")
    L.append("      // a block whose scores are all -inf for every row of the wave (a causal")
    L.append("      // mask's upper triangle) adds exactly nothing: skip its exp and P.V")
    L.append("      if (!__all(mb == (-__builtin_huge_valf()))) {")
    if D <= 64:
        # the V^T operands do not depend on the probabilities: read them now,
        # so their LDS latency hides behind the exponentials
        L.append(f"      v8 va[{D // 16}][{NT // 2}];")
        L.append("#pragma unroll")
        L.append(f"      for (int dt = 0; dt < {D // 16}; ++dt)")
        L.append("#pragma unroll")
        L.append(f"        for (int m = 0; m < {NT // 2}; ++m)")
        L.append(f"          va[dt][m] = *reinterpret_cast<const v8*>(vt + (dt * 16 + ql) * {PV} + g * 8 + m * 32);")
    L.append("      const float m_new = mlc::max_<float>(m_run, mb);")
    if FAST_SOFTMAX_MATH:
        # exponents in log2 units against the rounded RN(m log2 e): every exp
        # and every rescale of the row uses the same rounded values, so
        # their rounding is one common factor of o and l and cancels in o / l
        L.append("      const float ml_new = m_new * 0x1.715476p+0f;")
        L.append("      const float alpha = (m_run == (-__builtin_huge_valf())) ? 0.0f "
                 ": __builtin_amdgcn_exp2f(ml_run - ml_new);")
        L.append("      // a row with no finite score yet subtracts 0: its x are all -inf, exp gives 0")
        L.append("      const float ml_sub = m_new == (-__builtin_huge_valf()) ? 0.0f : ml_new;")
        exp_term = "__builtin_amdgcn_exp2f(__builtin_fmaf(x[t][i], 0x1.715476p+0f, -ml_sub))"
    else:
        L.append(f"      const float alpha = (m_run == (-__builtin_huge_valf())) ? 0.0f : {exp_}(m_run - m_new);")
        L.append("      // a row with no finite score yet subtracts 0: its x are all -inf, exp gives 0")
        L.append("      const float m_sub = m_new == (-__builtin_huge_valf()) ? 0.0f : m_new;")
        exp_term = f"{exp_}(x[t][i] - m_sub)"
    L.append(f"      v4 p[{NT}];")
    L.append("      float psum = 0.0f;")
    L.append("#pragma unroll")
    L.append(f"      for (int t = 0; t < {NT}; ++t)")
    L.append("#pragma unroll")
    L.append("        for (int i = 0; i < 4; ++i) {")
    L.append(f"          const float e = {exp_term};")
    L.append("          psum += e;")
    L.append(f"          p[t][i] = (e16)e;")
    L.append("        }")
    L.append("      l_run = l_run * alpha + psum;")
    L.append("      m_run = m_new;")
    if FAST_SOFTMAX_MATH:
        L.append("      ml_run = ml_new;")
    L.append(f"      v8 bq[{NT // 2}];")
    L.append("#pragma unroll")
    L.append(f"      for (int m = 0; m < {NT // 2}; ++m)")
    L.append("        bq[m] = v8{p[2 * m][0], p[2 * m][1], p[2 * m][2], p[2 * m][3], "
             "p[2 * m + 1][0], p[2 * m + 1][1], p[2 * m + 1][2], p[2 * m + 1][3]};")
    L.append("#pragma unroll")
    L.append(f"      for (int dt = 0; dt < {D // 16}; ++dt) o[dt] *= alpha;")
    if D <= 64:
        # the head-dim tiles' accumulations are independent; each still sums
        # its key pairs in order
        L.append("#pragma unroll")
        L.append(f"      for (int m = 0; m < {NT // 2}; ++m)")
        L.append("#pragma unroll")
        L.append(f"        for (int dt = 0; dt < {D // 16}; ++dt)")
        L.append("          o[dt] = mlc::mfma_16x16x32(va[dt][m], bq[m], o[dt]);")
    else:
        L.append("#pragma unroll")
        L.append(f"      for (int dt = 0; dt < {D // 16}; ++dt) {{")
        L.append(f"        const e16* vrow = vt + (dt * 16 + ql) * {PV} + g * 8;")
        L.append("#pragma unroll")
        L.append(f"        for (int m = 0; m < {NT // 2}; ++m) {{")
        L.append("          const v8 a = *reinterpret_cast<const v8*>(vrow + m * 32);")
        L.append("          o[dt] = mlc::mfma_16x16x32(a, bq[m], o[dt]);")
        L.append("        }")
        L.append("      }")
    L.append("      }")
    L.append("    }")
    L.append("    __syncthreads();  // every wave is done with this block's tiles")
    L.append(f"    if (b + 1 < {NB}) {{")
    L += ["    " + x for x in k_st + v_st]
    L.append("    }")
    L.append("    __syncthreads();")
    L.append("  }")
    L.append("  if (!active) return;")
    L.append("  l_run = mlc::xor32<mlc::OpSum>(mlc::xor16<mlc::OpSum>(l_run));")
    div = "* inv" if FAST_SOFTMAX_MATH else "/ l_run"
    if FAST_SOFTMAX_MATH:
        L.append("  const float inv = 1.0f / l_run;")
    omap = k.outputs[0].index
    parts = render_terms(axis_terms(omap, "idx"), BH * T * D, "f0", it)
    if omap.base:
        parts.append(f"({it}){omap.base}")
    L.append("#pragma unroll")
    L.append(f"  for (int dt = 0; dt < {D // 16}; ++dt) {{")
    L.append(f"    const v4 h = {{(e16)(o[dt][0] {div}), (e16)(o[dt][1] {div}), "
             f"(e16)(o[dt][2] {div}), (e16)(o[dt][3] {div})}};")
    L.append(f"    const {it} f0 = row * ({it}){D} + ({it})(dt * 16 + g * 4);")
    L.append(f"    *reinterpret_cast<v4*>(out0 + {join_offset(parts, it)}) = h;")
    L.append("  }")
    L.append("}")
    spec = LaunchSpec("", BH * NQB, THREADS, lds_bytes,
                      {"kind": "attention", "mode": "blocked", "heads": BH, "queries": T,
                       "keys": Tk, "head_dim": D, "queries_per_wg": QB, "key_block": KB})
    return "\n".join(L), spec
