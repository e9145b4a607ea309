// The HIP device the attention path renders on, beside `Machine` (Sources/LTXHardware/
// Machine.swift:12-30). Uncompiled here: the build image has no Swift toolchain.

import CLTXHip
import Foundation

/// One HIP device, measured at startup rather than assumed -- the same rule `Machine`
/// follows for the Mac: every field comes from the runtime (`ltx_device_query`).
///
/// Selection is explicit. Nothing in the package picks a HIP device by itself, just as no
/// render picks an attention path by itself (`Renderer.swift:113-131`): the caller names the
/// ordinal, `select` makes it current and records it, and the `.hip` attention path runs on
/// the selected device or refuses to run.
public struct HIPDevice: Sendable, Equatable, CustomStringConvertible {
    public let ordinal: Int32
    public let name: String
    /// `gcnArchName`, e.g. `gfx950:sramecc+:xnack-`.
    public let arch: String
    public let computeUnits: Int
    public let memoryBytes: UInt64
    public let clockKHz: Int
    public let ldsBytesPerCU: Int
    /// The library's kernels are built for gfx950 (MI355X) only.
    public let isSupported: Bool

    public var memoryGB: Double { Double(memoryBytes) / 1e9 }

    public var description: String {
        "\(name) [\(arch)] #\(ordinal): \(computeUnits) CUs, "
            + String(format: "%.0f GB", memoryGB)
    }

    /// Visible HIP devices (0 on a machine without one).
    public static var count: Int { Int(ltx_device_count()) }

    /// Describe device `ordinal`, or nil if there is no such device.
    public static func detect(ordinal: Int32 = 0) -> HIPDevice? {
        var info = ltx_device_info()
        guard ltx_device_query(ordinal, &info) == LTX_ATTN_OK else { return nil }
        func text<T>(_ tuple: T) -> String {
            withUnsafeBytes(of: tuple) { raw in
                String(decoding: raw.prefix { $0 != 0 }, as: UTF8.self)
            }
        }
        return HIPDevice(ordinal: info.ordinal, name: text(info.name), arch: text(info.arch),
                         computeUnits: Int(info.compute_units),
                         memoryBytes: UInt64(max(0, info.memory_bytes)),
                         clockKHz: Int(info.clock_khz), ldsBytesPerCU: Int(info.lds_bytes_per_cu),
                         isSupported: info.supported != 0)
    }

    public enum SelectionError: Error, CustomStringConvertible {
        case absent(Int32), unsupported(HIPDevice), runtime(String)
        public var description: String {
            switch self {
            case let .absent(o): return "no HIP device \(o)"
            case let .unsupported(d):
                return "\(d) is not gfx950; the attention kernels are built for MI355X only"
            case let .runtime(m): return m
            }
        }
    }

    private final class Selection: @unchecked Sendable {
        let lock = NSLock()
        var device: HIPDevice?
    }
    private static let selection = Selection()

    /// The device `select` made current, or nil before any selection.
    public static var selected: HIPDevice? {
        selection.lock.lock()
        defer { selection.lock.unlock() }
        return selection.device
    }

    /// Make device `ordinal` current for the calling thread and record it as the render's
    /// device. Refuses devices the kernels are not built for.
    @discardableResult
    public static func select(ordinal: Int32) throws -> HIPDevice {
        guard let d = detect(ordinal: ordinal) else { throw SelectionError.absent(ordinal) }
        guard d.isSupported else { throw SelectionError.unsupported(d) }
        let rc = cltx_set_device(ordinal)
        guard rc == 0 else { throw SelectionError.runtime(String(cString: cltx_error_string(rc))) }
        selection.lock.lock()
        selection.device = d
        selection.lock.unlock()
        return d
    }
}
