"""Hand-derived known answers of the Q4K sub-block fit, make_qkx1_quants(nmax 15, ntry 5),
and of one Q4K block built from such sub-blocks (the fit candle's BlockQ4K::from_float runs,
qwen3_next.rs:486-487 is the reference's call site). Shared by test_oracle_codecs.py, which
checks the oracle against them, and test_oracle_mutants.py, which checks that oracle builds
with one planted mistake each fail at least one of them.

Every value is IEEE f32 with one rounding per operation (no fused multiply-add), given as
its bit pattern. Rounding inside the fit is f32::round: halves away from zero.
The passes below list, per pass t: the codes L = clamp(round(iscale * (x - min)), 0, 15),
whether any code changed, sumlx = sum (x_i - min) * L_i (in element order), suml2 =
sum L_i^2, scale = sumlx / suml2, min = min(0, sum (x_i - scale * L_i) / n), and the next
iscale = 1 / scale. The loop stops after a pass in which no code changed, or after 5
passes; the result is (scale, -min).
"""

# ---- FIT_A: 4 elements, 3 passes, a rounding tie in pass 0.
# x = [0.75, 0.75, 4.5, 2.5]: min(x) = 0.75 > 0 -> min 0; iscale = 15 / 4.5 = 3.3333333
# (0x40555555).
# pass 0: iscale * x = [2.5, 2.5, 15, 8.333333]. 0.75 * 3.3333333 = 2.49999994 rounds to
#   the f32 2.5 exactly: a tie, so L = [3, 3, 15, 8] (half-even would give 2).
#   sumlx = 2.25 + 2.25 + 67.5 + 20 = 92, suml2 = 9 + 9 + 225 + 64 = 307,
#   scale = 92 / 307 = 0.29967427 (0x3e996ee8), sum = -0.19055414, min = -0.047638535
#   (0xbd4320a0), iscale = 3.3369565 (0x405590b2).
# pass 1: iscale * (x - min) = [2.661685, 2.661685, 15.175272, 8.501359],
#   L = [3, 3, 15, 9] (changed), sumlx = 95.929153 (0x42bfdbba), suml2 = 324,
#   scale = 0.29607764 (0x3e97977d), min = -0.095582306 (0xbdc3c0a8), iscale = 3.3774924.
# pass 2: iscale * (x - min) = [2.855948, 2.855948, 15.521545, 8.766560], L unchanged.
#   sumlx = ((2.536747 + 2.536747) + 68.933739) + 23.360241 = 97.367477 (0x42c2bc26)
#   in element order (the pairwise (a + b) + (c + d) gives 0x42c2bc25);
#   scale = 0.30051690 (0x3e99dd5a), min = -0.12887672 (0xbe03f842). No change: stop.
#   (A fourth pass would move scale and min again, to 0.30574051 / -0.16805387.)
FIT_A = ([0.75, 0.75, 4.5, 2.5], 0x3E99DD5A, 0x3E03F842)

# ---- FIT_B: 8 elements, codes change in all 5 passes (the pass limit decides).
# x = [-2, -1.25, 1, 5, 1, 1, 1.5, 2.5]: min -2, iscale = 15 / 7 = 2.1428571 (0x40092492).
# pass 0: iscale * (x + 2) = [0, 1.607143, 6.428571, 15, 6.428571, 6.428571, 7.5, 9.642857]
#   L = [0, 2, 6, 15, 6, 6, 8, 10], sumlx = 233.5, suml2 = 501,
#   scale = 0.46606785 (0x3eeea072), min = -1.9939497 (0xbfff39be).
# pass 1: L = [0, 2, 6, 15, 6, 6, 7, 10] (element 6: 7.496655 -> 7), sumlx = 229.68538
#   (0x4365af75), suml2 = 486, scale = 0.47260365 (0x3ef1f91b), min = -1.9781737 (0xbffd34cc).
# pass 2: L = [0, 2, 6, 15, 6, 6, 7, 9] (element 7: 9.475537 -> 9), sumlx = 224.38686
#   (0x43606309), suml2 = 467, scale = 0.48048577 (0x3ef6023b), min = -1.9693468 (0xbffc138e).
# pass 3: L = [0, 1, 6, 15, 6, 6, 7, 9] (element 1: 1.497124 -> 1), sumlx = 223.21736
#   (0x435f37a5), suml2 = 464, scale = 0.48107189 (0x3ef64f0e), min = -1.9129492 (0xbff4db85).
# pass 4: L = [0, 1, 6, 14, 6, 6, 7, 9] (element 3: 14.369888 -> 14), sumlx = 213.48450
#   (0x43557c08), suml2 = 435, scale = 0.49076897 (0x3efb4612), min = -1.9122101
#   (0xbff4c34d). Fifth pass done: stop.
#   (Four passes give 0x3ef64f0e / 0x3ff4db85; a sixth pass 0.49068573 / 1.9117002.)
FIT_B = ([-2.0, -1.25, 1.0, 5.0, 1.0, 1.0, 1.5, 2.5], 0x3EFB4612, 0x3FF4C34D)

# ---- FIT_P: a 32-element sub-block (the Q4K size), 3 passes. x = [6, 2, 2.25] then
# 29 x 1.0: min(x) = 1 > 0 -> min 0, iscale = 15 / 6 = 2.5; the 29 equal elements share
# one code, listed once as L[3].
# pass 0: iscale * x = [15, 5, 5.625, 2.5]: 2.5 is a tie -> 3; L[0:4] = [15, 5, 6, 3],
#   sumlx = 90 + 10 + 13.5 + 29 * 3 = 200.5, suml2 = 225 + 25 + 36 + 29 * 9 = 547,
#   scale = 0.36654478 (0x3ebbabc2), min = -0.067798823 (0xbd8ada1c).
# pass 1: L[0:4] = [15, 6, 6, 3] (element 1: 5.641... -> 6), sumlx = 210.22916
#   (0x43523aaa), suml2 = 558, scale = 0.37675476 (0x3ec0e600), min = -0.11562634 (0xbdeccd80).
# pass 2: codes unchanged; sumlx = 215.68138 (0x4357ae6f), suml2 = 558,
#   scale = 0.38652578 (0x3ec5e6b5), min = -0.15043563 (0xbe1a0bcc). Stop.
FIT_P = ([6.0, 2.0, 2.25] + [1.0] * 29, 0x3EC5E6B5, 0x3E1A0BCC)

# ---- FIT_Q: a 32-element sub-block, all positive (min stays clamped at 0), 5 passes.
# x = [2.75, 4.75, 5.25] then 29 x 0.5: min 0, iscale = 15 / 5.25 = 2.8571429.
# pass 0: L[0:4] = [8, 14, 15, 1] (0.5 * 2.857 = 1.43 -> 1), sumlx = 181.75, suml2 = 514,
#   scale = 0.35359922 (0x3eb50af5); sum > 0 -> min 0.
# pass 1: L[0:4] = [8, 13, 15, 1], sumlx = 177, suml2 = 487, scale = 0.36344969 (0x3eba1614).
# pass 2: L[0:4] = [8, 13, 14, 1], sumlx = 171.75, suml2 = 458, scale = 0.375 (0x3ec00000).
# pass 3: L[0:4] = [7, 13, 14, 1], sumlx = 169, suml2 = 443, scale = 0.38148984 (0x3ec352a3).
# pass 4: L[0:4] = [7, 12, 14, 1], sumlx = 164.25, suml2 = 418, scale = 0.39294258
#   (0x3ec92fc5); min 0 throughout, so -min = -0.0 (0x80000000). Pass limit: stop.
FIT_Q = ([2.75, 4.75, 5.25] + [0.5] * 29, 0x3EC92FC5, 0x80000000)

FITS = {"A": FIT_A, "B": FIT_B, "P": FIT_P, "Q": FIT_Q}

# ---- BLOCK_PQ: the Q4K block whose sub-blocks are P, Q, P, Q, P, Q, P, Q.
# max_scale = scale_Q = 0.39294258, max_min = -min_P = 0.15043563 (-min_Q = -0.0 < it).
# ls = round(63 / max_scale * scale_j): P 61.97 -> 62, Q -> 63; lm: P -> 63, Q -0.0 -> 0.
# Packed (j < 4: byte j = ls, byte j + 4 = lm; j >= 4: byte j + 4 = ls & 15 | (lm & 15) << 4
# and the top two bits of ls / lm into bits 6-7 of bytes j - 4 / j):
#   bytes 0-3 = 62 | 0xC0, 63 | 0xC0, ... = 254, 255, 254, 255; bytes 4-7 = 255, 0, 255, 0;
#   bytes 8-11 = 0xFE, 0x0F, 0xFE, 0x0F.
# d = f16(max_scale / 63) = 0x1E63, dmin = f16(max_min / 63) = 0x18E4.
# Nibbles: L = clamp(round((x + f32(dmin) * lm) / (f32(d) * ls)), 0, 15) per sub-block:
#   P (ls 62, lm 63): 6 -> 15, 2 -> 6, 2.25 -> 6, 1 -> 3;  Q (ls 63, lm 0): 2.75 -> 7,
#   4.75 -> 12, 5.25 -> 13, 0.5 -> 1. Byte 32c + l = L_P[l] | L_Q[l] << 4:
#   0x7F, 0xC6, 0xD6, then 29 x 0x13, repeated for the four 64-element chunks.
BLOCK_PQ_X = (FIT_P[0] + FIT_Q[0]) * 4
BLOCK_PQ_HEADER = [0x63, 0x1E, 0xE4, 0x18, 254, 255, 254, 255, 255, 0, 255, 0, 0xFE, 0x0F, 0xFE, 0x0F]
BLOCK_PQ_QS = ([0x7F, 0xC6, 0xD6] + [0x13] * 29) * 4
