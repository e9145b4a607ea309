// The `.hip` case of `DiTAttention.AttentionPath`: the arithmetic of DiTAttention.swift:358-381
// (q_norm / k_norm over the inner dim, the head split, split RoPE, SDPA with 1/sqrt(D)) on the
// selected MI355X through libltx_attn.so, returning the same `[B, heads, T, dimHead]` tensor
// the MLX paths produce, so the gate, merge and `to_out` that follow (:385-404) are unchanged.
//
// MLX arrays live in host memory where MLX has no GPU backend, so each call uploads its
// operands and downloads the result; a port that keeps its activations in HIP memory calls
// `HIPAttention.attend` on device tensors directly and moves nothing.
//
// Uncompiled here: the build image has no Swift toolchain.

import Foundation
import LTXAttention
import LTXHardware
import MLX

enum HIPDiTCore {
    private final class Contexts: @unchecked Sendable {
        let lock = NSLock()
        var byOrdinal: [Int32: HIPAttentionContext] = [:]
    }
    private static let contexts = Contexts()

    /// The context of the explicitly selected device (`HIPDevice.select`). A render that
    /// chose `.hip` without selecting a device fails here, by name, before any arithmetic.
    static func context() throws -> HIPAttentionContext {
        guard let device = HIPDevice.selected else {
            throw HIPAttention.Failure.noDevice(
                "attentionPath .hip needs a device: call HIPDevice.select(ordinal:) first")
        }
        contexts.lock.lock()
        defer { contexts.lock.unlock() }
        if let c = contexts.byOrdinal[device.ordinal] { return c }
        let c = try HIPAttentionContext(ordinal: device.ordinal)
        contexts.byOrdinal[device.ordinal] = c
        return c
    }

    /// The raw bf16 bit patterns of `a`, row-major.
    private static func bits(_ a: MLXArray) -> [UInt16] {
        a.asType(.bfloat16).view(dtype: .uint16).flattened().asArray(UInt16.self)
    }

    private static func upload(_ a: MLXArray, _ ctx: HIPAttentionContext) throws -> HIPBuffer {
        try bits(a).withUnsafeBytes { try ctx.upload($0) }
    }

    /// Tables `[1, heads, tokens, dimHead/2]` (what `DiTForward.rotaries` builds) as the
    /// library's batch-broadcast `[heads, tokens, dimHead/2]`.
    private static func table(_ t: MLXArray, heads: Int, tokens: Int, half: Int,
                              _ ctx: HIPAttentionContext) throws -> HIPBuffer {
        guard t.ndim == 4, t.dim(0) == 1, t.dim(1) == heads, t.dim(2) == tokens,
              t.dim(3) == half else {
            throw DiTAttention.Failure.shape("rotary table", got: t.shape,
                                             expected: "[1, \(heads), \(tokens), \(half)]")
        }
        return try upload(t, ctx)
    }

    /// Pre-norm projections `q` `[B, Tq, inner]`, `k`, `v` `[B, Tk, inner]`, the module's
    /// norm weights `[inner]` and its rotary pair(s) -> attention output `[B, heads, Tq, D]`.
    static func attend(q: MLXArray, k: MLXArray, v: MLXArray, qNorm: MLXArray, kNorm: MLXArray,
                       heads: Int, rotary: DiTAttention.Rotary?,
                       keyRotary: DiTAttention.Rotary?) throws -> MLXArray {
        let ctx = try context()
        let B = q.dim(0), Tq = q.dim(1), inner = q.dim(2), Tk = k.dim(1)
        let dimHead = inner / heads
        let (dq, dk, dv) = (try upload(q, ctx), try upload(k, ctx), try upload(v, ctx))
        let (wq, wk) = (try upload(qNorm, ctx), try upload(kNorm, ctx))
        var keep = [dq, dk, dv, wq, wk]
        var pe: HIPAttention.Rotary?
        var kpe: HIPAttention.Rotary?
        if let r = rotary {
            let c = try table(r.cos, heads: heads, tokens: Tq, half: dimHead / 2, ctx)
            let s = try table(r.sin, heads: heads, tokens: Tq, half: dimHead / 2, ctx)
            keep += [c, s]
            pe = HIPAttention.Rotary(cos: c.pointer, sin: s.pointer)
        }
        if let r = keyRotary {
            let c = try table(r.cos, heads: heads, tokens: Tk, half: dimHead / 2, ctx)
            let s = try table(r.sin, heads: heads, tokens: Tk, half: dimHead / 2, ctx)
            keep += [c, s]
            kpe = HIPAttention.Rotary(cos: c.pointer, sin: s.pointer)
        }
        let out = try HIPBuffer(bytes: B * Tq * inner * 2)
        let call = HIPAttention.Call(
            batch: Int32(B), heads: Int32(heads), headDim: Int32(dimHead),
            queryTokens: Int32(Tq), keyTokens: Int32(Tk),
            q: .merged(dq.pointer, tokens: Tq, inner: inner, headDim: dimHead),
            k: .merged(dk.pointer, tokens: Tk, inner: inner, headDim: dimHead),
            v: .merged(dv.pointer, tokens: Tk, inner: inner, headDim: dimHead),
            qNormWeight: wq.pointer, kNormWeight: wk.pointer,
            rotary: pe, keyRotary: kpe,
            out: out.pointer,
            outStrides: (Int64(Tq * inner), Int64(inner), Int64(dimHead)))
        let bytes = try HIPAttention.workspaceBytes(call)
        let ws = try ctx.workspace(bytes: bytes)
        try HIPAttention.attend(call, workspace: ws?.pointer, workspaceBytes: bytes,
                                stream: ctx.stream)
        var host = [UInt16](repeating: 0, count: B * Tq * inner)
        try host.withUnsafeMutableBytes { try ctx.download(out, into: $0) }
        withExtendedLifetime(keep) {}
        // [B, Tq, inner] -> [B, heads, Tq, dimHead], the layout `split` gives (:346-349)
        return MLXArray(host).reshaped([B, Tq, heads, dimHead]).view(dtype: .bfloat16)
            .transposed(0, 2, 1, 3)
    }
}
