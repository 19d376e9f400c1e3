"""The reference graph's forward composed only from the net.h launchers of the C ABI, in the order
src/dit_fwd.cpp:104-304 issues them, against the oracle's restatement of the same graph
(orc_ref_dit_forward) at the reference's 8 s geometry (T = 172 latent, C = 64 clip, TS = 154 text
rows, H = 1024, SwiGLU F = 2816, 7 joint + 14 fused blocks).

This is the drop-in a maintainer gets by keeping src/dit_fwd.cpp and binding its Runtime calls and
named-kernel dispatches to tsn_gemm, tsn_gemv, tsn_conv1d, tsn_adaln_ln, tsn_qkv_split3,
tsn_rms_head, tsn_rope_pairs, tsn_attention, tsn_gate_add, tsn_swiglu, tsn_silu, tsn_add*,
tsn_copy: one forward per CFG arm (src/pipeline.cpp:146-147), f32 activations, f16 GEMM and conv
weights, f32 vectors, the element-interleaved qkv projection de-interleaved by qkv_split3.
Bars: velocity rel-L2 <= 1e-3 per evaluation and every stream after every block <= 2e-3.
"""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu

F32, F16 = 0, 1


class _At:
    """a device address inside an array (the reference's (char *) buf.p + offset)"""

    def __init__(self, arr, elems=0):
        self.p = arr.offset(elems)


class LauncherDit:
    """src/dit_fwd.cpp's forward over the launcher surface. Weights as WeightSet::load leaves them
    (src/net.mm:126-173): matrices f16, 1-D tensors f32; conv weights additionally prepared once
    with tsn_conv1d_prepare, the load-time step the implicit-GEMM conv needs."""

    def __init__(self, tsn, rt, spec, w_bf16):
        self.rt, self.s = rt, spec
        H, T, C, TS, F = spec.H, spec.T, spec.C, spec.TS, spec.F
        self.W = {}
        w32 = tsn.bf16_to_f32(w_bf16)
        conv_taps = {}
        for name, numel, off in tsn.ref_manifest(spec):
            v = w32[off:off + numel]
            if name.endswith("weight") and numel > spec.HD:
                # bf16 -> f16 (exact in f16's normal range; numpy rounds the few subnormal results
                # to nearest where the reference's converter truncates)
                self.W[name] = rt.array(v.astype(np.float16))
            else:
                self.W[name] = rt.array(v)
        # conv weights [OC][IC][K] (the latent / clip out-projection and FFNs, input projection, final conv)
        for name, numel, _ in tsn.ref_manifest(spec):
            K = self._conv_k(name)
            if K:
                OC, IC = self._conv_oc_ic(name)
                assert OC * IC * K == numel, name
                Wp = rt.empty((rt.conv1d_prepared_bytes(F16, OC, IC, K),), np.uint8)
                rt.conv1d_prepare(self.W[name], F16, Wp, OC, IC, K)
                conv_taps[name] = Wp
        self.Wp = conv_taps
        S = T + C + TS
        e = rt.empty
        self.te_out, self.te_scr, self.global_c, self.gc_pre = e((H,)), e((H,)), e((H,)), e((H,))
        self.extc, self.extc_silu, self.x_in = e((T, H)), e((T, H)), e((T, H))
        self.sc_f1, self.sc_f3 = e((S, max(F, H))), e((S, max(F, H)))
        self.sc_qkv, self.jointq = e((S, 3 * H)), e((S, 3 * H))
        self.joint_att, self.sc_l1, self.sc_r = e((S, H)), e((S, H)), e((S, H))
        self.mod_lat, self.mod_clip, self.mod_text = e((T, 6 * H)), e((6 * H,)), e((6 * H,))
        self.mod_fin = e((T, 2 * H))
        self.clip_s, self.text_s = e((C, H)), e((TS, H))
        self.pos_lat = rt.array(np.arange(T, dtype=np.int32))
        self.pos_clip = rt.array(np.arange(C, dtype=np.int32))

    def _conv_k(self, name):
        """kernel width of a conv weight (src/dit_fwd.cpp:56-61,73-76,142-149,302-303), 0 otherwise"""
        if not name.endswith("weight"):
            return 0
        if name == "final_layer.conv.weight":
            return 7
        if name.startswith("audio_input_proj"):
            return 3
        if ".text_block." in name:
            return 0
        return 3 if (".linear1." in name or ".ffn." in name) else 0

    def _conv_oc_ic(self, name):
        s = self.s
        if name == "audio_input_proj.0.weight":
            return s.H, s.latent
        if name == "final_layer.conv.weight":
            return s.latent, s.H
        if name.endswith("w2.weight"):
            return s.H, s.F
        if name.endswith("w1.weight") or name.endswith("w3.weight"):
            return s.F, s.H
        return s.H, s.H   # linear1

    def conv(self, name, bias, x, y, T, IC, OC, K, pad, dil):
        # src/dit_fwd.cpp:12-15: rt.conv(true, w, b, x, y, T, T, IC, OC, K, 1, pad, dil)
        self.rt.conv1d(F16, self.Wp[name], bias, x, y, T, T, IC, OC, K, 1, pad, dil)

    def pre_attn(self, bp, x, mod, per_row, rows, row_off, qkv_dst, pos, fscale, is_text, chunks=6):
        # src/dit_fwd.cpp:24-49
        rt, s, W, H = self.rt, self.s, self.W, self.s.H
        rt.adaln_ln(x, mod, self.sc_f1, F32, rows, H, 1 if per_row else 0, chunks, 0, 1e-5)
        rt.gemm(F16, W[bp + ".attn.qkv.weight"], self.sc_f1, F32, qkv_dst, F32, W[bp + ".attn.qkv.bias"],
                rows, 3 * H, H, H, H, 3 * H)
        rt.qkv_split3(qkv_dst, self.sc_qkv, rows, H, row_off)
        rt.rms_head(self.sc_qkv, W[bp + ".attn.q_norm.weight"], rows, s.NH, 3 * H, s.HD, 0, row_off, 1e-6)
        rt.rms_head(self.sc_qkv, W[bp + ".attn.k_norm.weight"], rows, s.NH, 3 * H, s.HD, H, row_off, 1e-6)
        if not is_text:
            rt.rope_pairs(self.sc_qkv, pos, rows, s.NH, 3 * H, s.HD, 0, row_off, fscale, s.rope_theta)
            rt.rope_pairs(self.sc_qkv, pos, rows, s.NH, 3 * H, s.HD, H, row_off, fscale, s.rope_theta)

    def post_attn(self, bp, x, attn_out, mod, per_row, rows, is_text):
        # src/dit_fwd.cpp:51-81
        rt, W, H, F = self.rt, self.W, self.s.H, self.s.F
        pr = 1 if per_row else 0
        if is_text:
            rt.gemm(F16, W[bp + ".linear1.weight"], attn_out, F32, self.sc_l1, F32, W[bp + ".linear1.bias"],
                    rows, H, H)
        else:
            self.conv(bp + ".linear1.weight", W[bp + ".linear1.bias"], attn_out, self.sc_l1, rows, H, H, 3, 1, 1)
        rt.gate_add(x, self.sc_l1, mod, x, rows, H, pr, 6, 2)
        rt.adaln_ln(x, mod, self.sc_r, F32, rows, H, pr, 6, 3 * H, 1e-5)
        if is_text:
            rt.gemm(F16, W[bp + ".ffn.w1.weight"], self.sc_r, F32, self.sc_f1, F32, None, rows, F, H)
            rt.gemm(F16, W[bp + ".ffn.w3.weight"], self.sc_r, F32, self.sc_f3, F32, None, rows, F, H)
            rt.swiglu(self.sc_f1, self.sc_f3, self.sc_f1, rows * F)
            rt.gemm(F16, W[bp + ".ffn.w2.weight"], self.sc_f1, F32, self.sc_f3, F32, None, rows, H, F)
        else:
            self.conv(bp + ".ffn.w1.weight", None, self.sc_r, self.sc_f1, rows, H, F, 3, 1, 1)
            self.conv(bp + ".ffn.w3.weight", None, self.sc_r, self.sc_f3, rows, H, F, 3, 1, 1)
            rt.swiglu(self.sc_f1, self.sc_f3, self.sc_f1, rows * F)
            self.conv(bp + ".ffn.w2.weight", None, self.sc_f1, self.sc_f3, rows, F, H, 3, 1, 1)
        rt.gate_add(x, self.sc_f3, mod, x, rows, H, pr, 6, 5)

    def attention(self, S):
        # src/dit_fwd.cpp:83-102 (AttnP: ld 3H, ldo H, q/k/v at 0/H/2H, scale 1/sqrt(hd))
        s = self.s
        self.rt.attention(self.sc_qkv, self.joint_att, S, s.NH, s.HD, 3 * s.H, s.H, 0, s.H, 2 * s.H, 0,
                          float(np.float32(1.0) / np.sqrt(np.float32(s.HD))))

    def forward(self, x, t, text_pp, gcmlp, flow, clip_pp, sync_gather, taps=None):
        # src/dit_fwd.cpp:104-304 for one CFG arm
        rt, s, W = self.rt, self.s, self.W
        H, T, C, TS, F, L = s.H, s.T, s.C, s.TS, s.F, s.latent
        half = H // 2
        k = np.arange(half, dtype=np.float32)
        fr = np.float32(10000.0 / s.t_max_period) * np.power(np.float32(10000.0), np.float32(-2.0) * k / np.float32(H))
        temb = np.concatenate([np.cos(np.float32(t) * fr), np.sin(np.float32(t) * fr)]).astype(np.float32)
        in_temb = rt.array(temb)
        rt.gemv(W["t_embed.mlp.0.weight"], F16, in_temb, self.te_out, W["t_embed.mlp.0.bias"], H, H, H)
        rt.silu(self.te_out, H)
        rt.gemv(W["t_embed.mlp.2.weight"], F16, self.te_out, self.te_scr, W["t_embed.mlp.2.bias"], H, H, H)
        rt.add_(gcmlp, self.te_scr, self.global_c, H)
        rt.copy(self.te_scr, self.te_out, H)
        rt.add_bcast_col(sync_gather, self.global_c, self.extc, T, H)
        rt.copy(self.extc, self.extc_silu, T * H)
        rt.silu(self.extc_silu, T * H)
        rt.copy(self.global_c, self.gc_pre, H)
        rt.silu(self.global_c, H)
        self.conv("audio_input_proj.0.weight", W["audio_input_proj.0.bias"], x, self.x_in, T, L, H, 3, 1, 1)
        rt.silu(self.x_in, T * H)
        self.conv("audio_input_proj.2.w1.weight", None, self.x_in, self.sc_f1, T, H, F, 3, 1, 1)
        self.conv("audio_input_proj.2.w3.weight", None, self.x_in, self.sc_f3, T, H, F, 3, 1, 1)
        rt.swiglu(self.sc_f1, self.sc_f3, self.sc_f1, T * F)
        self.conv("audio_input_proj.2.w2.weight", None, self.sc_f1, self.x_in, T, F, H, 3, 1, 1)
        rt.copy(clip_pp, self.clip_s, C * H)
        rt.copy(text_pp, self.text_s, TS * H)
        lat = self.x_in
        S = T + C + TS
        for i in range(s.n_joint):
            pre_only = i == s.n_joint - 1
            jb = "joint_blocks.%d" % i
            rt.gemm(F16, W[jb + ".latent_block.adaLN_modulation.1.weight"], self.extc_silu, F32, self.mod_lat, F32,
                    W[jb + ".latent_block.adaLN_modulation.1.bias"], T, 6 * H, H)
            self.pre_attn(jb + ".latent_block", lat, self.mod_lat, True, T, 0, self.jointq, self.pos_lat, 1.0,
                          False, 6)
            ct = 2 if pre_only else 6
            rt.gemv(W[jb + ".clip_block.adaLN_modulation.1.weight"], F16, self.global_c, self.mod_clip,
                    W[jb + ".clip_block.adaLN_modulation.1.bias"], ct * H, H, H)
            self.pre_attn(jb + ".clip_block", self.clip_s, self.mod_clip, False, C, T, _At(self.jointq, T * 3 * H),
                          self.pos_clip, float(np.float32(T) / np.float32(C)), False, ct)
            rt.gemv(W[jb + ".text_block.adaLN_modulation.1.weight"], F16, self.global_c, self.mod_text,
                    W[jb + ".text_block.adaLN_modulation.1.bias"], ct * H, H, H)
            self.pre_attn(jb + ".text_block", self.text_s, self.mod_text, False, TS, T + C,
                          _At(self.jointq, (T + C) * 3 * H), None, 1.0, True, ct)
            self.attention(S)
            self.post_attn(jb + ".latent_block", lat, self.joint_att, self.mod_lat, True, T, False)
            if not pre_only:
                self.post_attn(jb + ".clip_block", self.clip_s, _At(self.joint_att, T * H), self.mod_clip, False, C,
                               False)
                self.post_attn(jb + ".text_block", self.text_s, _At(self.joint_att, (T + C) * H), self.mod_text,
                               False, TS, True)
            if taps is not None:
                taps.append(self._streams(lat))
        for i in range(s.n_fused):
            fb = "fused_blocks.%d" % i
            rt.gemm(F16, W[fb + ".adaLN_modulation.1.weight"], self.extc_silu, F32, self.mod_lat, F32,
                    W[fb + ".adaLN_modulation.1.bias"], T, 6 * H, H)
            self.pre_attn(fb, lat, self.mod_lat, True, T, 0, self.jointq, self.pos_lat, 1.0, False, 6)
            self.attention(T)
            self.post_attn(fb, lat, self.joint_att, self.mod_lat, True, T, False)
            if taps is not None:
                taps.append(self._streams(lat))
        rt.gemm(F16, W["final_layer.adaLN_modulation.1.weight"], self.extc_silu, F32, self.mod_fin, F32,
                W["final_layer.adaLN_modulation.1.bias"], T, 2 * H, H)
        rt.adaln_ln(lat, self.mod_fin, self.sc_l1, F32, T, H, 1, 2, 0, 1e-5)
        self.conv("final_layer.conv.weight", W["final_layer.conv.bias"], self.sc_l1, flow, T, H, L, 7, 3, 1)

    def _streams(self, lat):
        self.rt.sync()
        return np.concatenate([lat.numpy(), self.clip_s.numpy(), self.text_s.numpy()], axis=0)


def test_reference_graph_from_launchers(tsn, rt, orc):
    spec = tsn.ref_spec_for_duration(8, 2)
    w16 = tsn.ref_synth_weights(spec, 4242, 1.0)
    m = LauncherDit(tsn, rt, spec, w16)
    inp = tsn.ref_synth_inputs(spec, 4242)
    T, C, TS, H, L = spec.T, spec.C, spec.TS, spec.H, spec.latent
    v = np.zeros((spec.B, T, L), np.float32)
    taps = []
    for b in range(spec.B):
        dev = {k: rt.array(inp[k][b]) for k in ("x", "clip_pp", "text_pp", "gcmlp", "sync_gather")}
        flow = rt.empty((T, L))
        tb = []
        m.forward(dev["x"], float(inp["t"][b]), dev["text_pp"], dev["gcmlp"], flow, dev["clip_pp"],
                  dev["sync_gather"], tb)
        rt.sync()
        v[b] = flow.numpy()
        taps.append(tb)
    vr, tr = orc.ref_dit_forward(spec.as_dict(), tsn.bf16_to_f32(w16), taps=True, **inp)
    err = rel_l2(v, vr)
    nblk = spec.n_joint + spec.n_fused
    blk = [rel_l2(np.stack([taps[b][i] for b in range(spec.B)]), tr[i]) for i in range(nblk)]
    lat = [rel_l2(np.stack([taps[b][i][:T] for b in range(spec.B)]), tr[i][:, :T]) for i in range(nblk)]
    print("launcher-composed reference graph: velocity rel-L2 %.3g; worst block %.3g (latent %.3g)"
          % (err, max(blk), max(lat)))
    assert err <= 1e-3
    assert max(blk) <= 2e-3 and max(lat) <= 2e-3
