// Admission for the `.hip` attention path, beside `MemoryPlan` (Sources/LTXHardware/
// MemoryPlan.swift:56-72): whether the selected HIP device holds what the path puts on it, from
// the library's own workspace sizing and the device's measured free memory.
//
// Uncompiled here: the build image has no Swift toolchain.

import CLTXHip
import Foundation

/// What the `.hip` path holds on the device for a render, and whether the selected device has
/// it free.
///
/// The MLX weights and activations stay where MLX keeps them; on the device the path holds one
/// context (`HIPAttentionContext`): an operand arena as large as the largest call's inputs and
/// output, and a workspace as large as the largest call's `ltx_attn_workspace_bytes`. Both
/// grow to the largest call and stay, so the plan is the maximum over the calls a render
/// makes. The phases do not overlap -- the text encoder's 48 layers run before sampling, as in
/// `MemoryPlan` -- so the device need is the larger of the two phases.
public struct HIPMemoryPlan: Sendable, Equatable {
    public enum Phase: String, Sendable, CaseIterable {
        case textEncode, sampling
    }

    /// One attention call of a phase: the library's argument shapes.
    struct Call {
        var name: String
        var batch: Int, heads: Int, headDim: Int, queryTokens: Int, keyTokens: Int
        var queryRotary: Bool, keyRotary: Bool
    }

    public let videoTokens: Int
    public let audioTokens: Int
    /// Device bytes per phase: arena + workspace of its largest call.
    public let phaseBytes: [Phase: UInt64]
    public let peakBytes: UInt64
    /// `hipMemGetInfo`'s free bytes on the selected device, measured when planned.
    public let availableBytes: UInt64
    public let headroomBytes: Int64
    public let marginFraction: Double

    public var fits: Bool { headroomBytes > 0 }

    public struct Refusal: Error, CustomStringConvertible {
        public let plan: HIPMemoryPlan?
        public let reason: String
        public var description: String {
            reason + (plan.map { "\n" + $0.explanation } ?? "")
        }
    }

    static func aligned(_ n: Int) -> Int { (n + 255) / 256 * 256 }

    /// Workspace of one DiT attention call (`ltx_attn_workspace_bytes`: a pure host function
    /// of the shapes; the pointers are placeholders it only checks for alignment).
    static func workspace(_ c: Call) -> Int {
        let inner = Int64(c.heads * c.headDim)
        let fake = UnsafeMutableRawPointer(bitPattern: 0x1_0000)!
        var a = ltx_attn_args()
        ltx_attn_args_init(&a)
        a.B = Int32(c.batch); a.H = Int32(c.heads); a.D = Int32(c.headDim)
        a.Lq = Int32(c.queryTokens); a.Lk = Int32(c.keyTokens)
        a.q = UnsafeRawPointer(fake); a.k = UnsafeRawPointer(fake); a.v = UnsafeRawPointer(fake)
        a.q_bs = Int64(c.queryTokens) * inner; a.q_rs = inner; a.q_hs = Int64(c.headDim)
        a.k_bs = Int64(c.keyTokens) * inner; a.k_rs = inner; a.k_hs = Int64(c.headDim)
        a.v_bs = a.k_bs; a.v_rs = inner; a.v_hs = Int64(c.headDim)
        a.q_norm_w = UnsafeRawPointer(fake); a.k_norm_w = UnsafeRawPointer(fake)
        if c.queryRotary { a.q_cos = UnsafeRawPointer(fake); a.q_sin = UnsafeRawPointer(fake) }
        if c.keyRotary { a.k_cos = UnsafeRawPointer(fake); a.k_sin = UnsafeRawPointer(fake) }
        a.scale = Float(1.0 / Double(c.headDim).squareRoot())
        a.out = fake
        a.o_bs = a.q_bs; a.o_rs = inner; a.o_hs = Int64(c.headDim)
        return Int(ltx_attn_workspace_bytes(&a))
    }

    /// Operand arena of one DiT attention call, laid out as `HIPDiTCore.attend` lays it out:
    /// q, k, v, both norm weights, the tables it is given, the output (bf16, 256-byte aligned).
    static func arena(_ c: Call) -> Int {
        let inner = c.heads * c.headDim
        let nq = c.batch * c.queryTokens * inner, nk = c.batch * c.keyTokens * inner
        var bytes = aligned(2 * nq) + 2 * aligned(2 * nk) + 2 * aligned(2 * inner)
        if c.queryRotary { bytes += 2 * aligned(c.heads * c.queryTokens * c.headDim) }
        if c.keyRotary { bytes += 2 * aligned(c.heads * c.keyTokens * c.headDim) }
        return bytes + aligned(2 * nq)
    }

    /// The six calls of a DiT block (`DiTBlock.swift:343-438`) at a render's token counts: 32
    /// heads, video width 4096 (D 128), audio and cross-modal width 2048 (D 64)
    /// (`TransformerTopology.swift:51`, `:134-143`), the text keys unmasked.
    static func blockCalls(videoTokens: Int, audioTokens: Int, textTokens: Int,
                           batch: Int) -> [Call] {
        [
            Call(name: "attn1", batch: batch, heads: 32, headDim: 128, queryTokens: videoTokens,
                 keyTokens: videoTokens, queryRotary: true, keyRotary: false),
            Call(name: "audio_attn1", batch: batch, heads: 32, headDim: 64,
                 queryTokens: audioTokens, keyTokens: audioTokens, queryRotary: true,
                 keyRotary: false),
            Call(name: "attn2", batch: batch, heads: 32, headDim: 128, queryTokens: videoTokens,
                 keyTokens: textTokens, queryRotary: false, keyRotary: false),
            Call(name: "audio_attn2", batch: batch, heads: 32, headDim: 64,
                 queryTokens: audioTokens, keyTokens: textTokens, queryRotary: false,
                 keyRotary: false),
            Call(name: "audio_to_video_attn", batch: batch, heads: 32, headDim: 64,
                 queryTokens: videoTokens, keyTokens: audioTokens, queryRotary: true,
                 keyRotary: true),
            Call(name: "video_to_audio_attn", batch: batch, heads: 32, headDim: 64,
                 queryTokens: audioTokens, keyTokens: videoTokens, queryRotary: true,
                 keyRotary: true),
        ]
    }

    /// The text encoder's attention (`GemmaTextEncoder+HIP.swift`): the full layers are the
    /// larger (16 query heads of 512 over one KV head shared as V), fp32 output.
    static func textEncodeBytes(textTokens: Int) -> Int {
        let T = textTokens, Hq = 16, D = 512
        let fake = UnsafeMutableRawPointer(bitPattern: 0x1_0000)!
        var a = ltx_gemma_attn_args()
        a.B = 1; a.T = Int32(T); a.Hq = Int32(Hq); a.Hkv = 1; a.D = Int32(D)
        a.q = UnsafeRawPointer(fake); a.k = UnsafeRawPointer(fake); a.v = UnsafeRawPointer(fake)
        a.q_rs = Int64(Hq * D); a.k_rs = Int64(D); a.v_rs = Int64(D)
        a.q_bs = a.q_rs * Int64(T); a.k_bs = a.k_rs * Int64(T); a.v_bs = a.k_bs
        a.q_norm_w = UnsafeRawPointer(fake); a.k_norm_w = UnsafeRawPointer(fake)
        a.eps = 1e-6; a.scale = 1.0
        a.cos = UnsafePointer(fake.assumingMemoryBound(to: Float.self))
        a.sin = a.cos
        a.out = fake.assumingMemoryBound(to: Float.self)
        a.o_rs = Int64(Hq * D); a.o_bs = a.o_rs * Int64(T)
        let workspace = Int(ltx_gemma_attn_workspace_bytes(&a))
        let arena = aligned(2 * T * Hq * D) + aligned(2 * T * D) + 2 * aligned(2 * D)
            + 2 * aligned(4 * T * D / 2) + aligned(4 * T * Hq * D)
        return workspace + arena
    }

    /// The plan for a render of `videoTokens` (with any reference tokens) and `audioTokens`,
    /// CFG batch 2, against `availableBytes` of free device memory.
    public static func plan(videoTokens: Int, audioTokens: Int, textTokens: Int = 1024,
                            batch: Int = 2, availableBytes: UInt64,
                            marginFraction: Double = 0.15) -> HIPMemoryPlan {
        let calls = blockCalls(videoTokens: videoTokens, audioTokens: audioTokens,
                               textTokens: textTokens, batch: batch)
        let sampling = UInt64(calls.map(workspace).max() ?? 0) + UInt64(calls.map(arena).max() ?? 0)
        let phases: [Phase: UInt64] = [
            .textEncode: UInt64(textEncodeBytes(textTokens: textTokens)),
            .sampling: sampling,
        ]
        let peak = phases.values.max() ?? 0
        let withMargin = UInt64(Double(peak) * (1.0 + marginFraction))
        return HIPMemoryPlan(videoTokens: videoTokens, audioTokens: audioTokens,
                             phaseBytes: phases, peakBytes: peak, availableBytes: availableBytes,
                             headroomBytes: Int64(availableBytes) - Int64(withMargin),
                             marginFraction: marginFraction)
    }

    /// Plan against the selected device's free memory, measured now, and refuse a render that
    /// does not fit -- before any weight is loaded, as `MemoryPlan` refuses one for the Mac.
    @discardableResult
    public static func admit(videoTokens: Int, audioTokens: Int, textTokens: Int = 1024,
                             batch: Int = 2, marginFraction: Double = 0.15) throws
        -> HIPMemoryPlan {
        guard HIPDevice.selected != nil else {
            throw Refusal(plan: nil, reason: "attentionPath .hip needs a device: call "
                          + "HIPDevice.select(ordinal:) first")
        }
        var free = 0, total = 0
        let rc = cltx_mem_info(&free, &total)
        guard rc == 0 else {
            throw Refusal(plan: nil, reason: "hipMemGetInfo: "
                          + String(cString: cltx_error_string(rc)))
        }
        let p = plan(videoTokens: videoTokens, audioTokens: audioTokens,
                     textTokens: textTokens, batch: batch, availableBytes: UInt64(free),
                     marginFraction: marginFraction)
        guard p.fits else {
            throw Refusal(plan: p, reason: "the .hip attention path does not fit the selected "
                          + "HIP device")
        }
        return p
    }

    public var explanation: String {
        var lines = [String(format: "  video tokens   %d, audio tokens %d (.hip attention)",
                            videoTokens, audioTokens)]
        for phase in Phase.allCases {
            let b = phaseBytes[phase] ?? 0
            let name = phase.rawValue.padding(toLength: 14, withPad: " ", startingAt: 0)
            lines.append(String(format: "  %@ %8.2f GB%@", name, Double(b) / 1e9,
                                b == peakBytes ? "   <- peak" : ""))
        }
        lines.append(String(format: "  device free    %8.2f GB", Double(availableBytes) / 1e9))
        lines.append(String(format: "  headroom       %+8.2f GB after a %.0f%% margin",
                            Double(headroomBytes) / 1e9, marginFraction * 100))
        return lines.joined(separator: "\n")
    }
}
