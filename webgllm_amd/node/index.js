'use strict'
/**
 * HipGpu: the reference's GPU-backend contract (class Gpu,
 * src/gpu/gl.ts:47; PendingRead and GpuError, src/gpu/types.ts:12-14) over
 * the N-API addon webgllm_hip.node and libwebgllm_hip.so, plus an `ops`
 * object of native kernels, which an engine detects as it detects
 * `nativeProgram` on WebGPU (src/engine.ts:5039). A texture is a flat
 * device buffer with the same bytes, rows of `width` texels.
 *
 * CommonJS, so that Node 12 loads it as it is.
 */
const path = require('path')

const addon = require(path.join(__dirname, 'webgllm_hip.node'))

/** The WebGL 2 formats the engine makes textures in (src/gpu/types.ts:21-41). */
const GL = {
  RGBA32F: 0x8814,
  RGBA4: 0x8056,
  RGBA8: 0x8058,
  RGBA16F: 0x881a,
  R32F: 0x822e,
  R32UI: 0x8236,
  R8UI: 0x8232,
  RGBA32UI: 0x8d70,
  RGBA8UI: 0x8d7c,
  RGBA8I: 0x8d8e
}

/** Bytes a texel of each format holds. */
const TEXEL_BYTES = {
  [GL.RGBA32F]: 16,
  [GL.RGBA4]: 2,
  [GL.RGBA8]: 4,
  [GL.RGBA16F]: 8,
  [GL.R32F]: 4,
  [GL.R32UI]: 4,
  [GL.R8UI]: 1,
  [GL.RGBA32UI]: 16,
  [GL.RGBA8UI]: 4,
  [GL.RGBA8I]: 4
}

class GpuError extends Error {}

/** The addon's errors as GpuError, keeping the status name and number. */
function rethrow (e) {
  if (e && e.name === 'GpuError' && !(e instanceof GpuError)) {
    const g = new GpuError(e.message)
    g.code = e.code
    g.status = e.status
    throw g
  }
  throw e
}

function call (fn, ...args) {
  try {
    return fn(...args)
  } catch (e) {
    rethrow(e)
  }
}

function bytesOf (view) {
  return Buffer.from(view.buffer, view.byteOffset, view.byteLength)
}

/** A rectangle's texels as floats, out of the rows [rect.y, rect.y + height) read whole. */
function cut (ab, t, rect, texel) {
  if (rect.x === 0 && rect.width === t.width) return new Float32Array(ab)
  const out = new Uint8Array(rect.width * rect.height * texel)
  const all = new Uint8Array(ab)
  for (let r = 0; r < rect.height; r++) {
    const s = (r * t.width + rect.x) * texel
    out.set(all.subarray(s, s + rect.width * texel), r * rect.width * texel)
  }
  return new Float32Array(out.buffer)
}

class HipGpu {
  constructor (device = 0) {
    this.ctx = call(addon.ctxCreate, device)
    const lim = call(addon.ctxLimits, this.ctx)
    // the reference's limits (gl.ts:131-140): buffers have no 2D size limit
    this.limits = {
      maxTextureSize: 1 << 30,
      maxDrawBuffers: 8,
      maxTextureUnits: 64,
      renderer: lim.renderer,
      computeUnits: lim.computeUnits,
      globalBytes: lim.globalBytes
    }
    this.nextId = 1
    this.live = new Set()
    this.lost = false
  }

  /** Device bytes the textures hold (Gpu.bytes). */
  get bytes () { return call(addon.bytesLive, this.ctx) }

  isLost () { return this.lost }

  /** Gpu.texture (gl.ts:263-305). `data.pixels`: the texels' bytes, row-major. */
  texture (internal, width, height, data) {
    if (!(width >= 1 && height >= 1)) throw new GpuError(`A ${width}×${height} texture is empty.`)
    const bytes = width * height * (TEXEL_BYTES[internal] || 16)
    let init = null
    if (data) {
      init = bytesOf(data.pixels)
      if (init.length !== bytes) throw new GpuError(`${init.length} bytes for a ${bytes}-byte texture.`)
    }
    const tex = call(addon.bufCreate, this.ctx, bytes, init)
    const t = { id: this.nextId++, tex, width, height, internal, bytes }
    this.live.add(t)
    return t
  }

  /** Gpu.write (gl.ts:354-374): the rectangle's texels, row by row. */
  write (target, rect, data) {
    const texel = target.bytes / (target.width * target.height)
    const src = bytesOf(data.pixels)
    const rowBytes = rect.width * texel
    if (src.length < rowBytes * rect.height) throw new GpuError('Too few bytes for the rectangle.')
    if (rect.x === 0 && rect.width === target.width) {
      call(addon.bufWrite, this.ctx, target.tex, rect.y * rowBytes, src.subarray(0, rowBytes * rect.height))
      return
    }
    for (let r = 0; r < rect.height; r++) {
      const off = ((rect.y + r) * target.width + rect.x) * texel
      call(addon.bufWrite, this.ctx, target.tex, off, src.subarray(r * rowBytes, (r + 1) * rowBytes))
    }
  }

  /** Gpu.zero (gl.ts:710-726). */
  zero (t) { call(addon.bufZero, this.ctx, t.tex) }

  /** Gpu.delete (gl.ts:448-461). */
  delete (t) {
    if (!this.live.delete(t)) return
    call(addon.bufDelete, this.ctx, t.tex)
  }

  /**
   * Gpu.readStart (gl.ts:740-782): the rectangle's bytes read back behind
   * the work already queued, as a PendingRead: call it for a Promise of the
   * floats (polling the fence between event-loop turns), or cancel it.
   */
  readStart (t, rect = { x: 0, y: 0, width: t.width, height: t.height }) {
    const texel = t.bytes / (t.width * t.height)
    const band = rect.height * t.width * texel
    const fence = call(addon.readStart, this.ctx, t.tex, rect.y * t.width * texel, band)
    let done = false
    const wait = async () => {
      if (done) throw new Error('This read was cancelled or already taken.')
      while (!call(addon.fenceReady, fence)) await new Promise((resolve) => setImmediate(resolve))
      done = true
      return cut(call(addon.readFinish, fence, band), t, rect, texel)
    }
    return Object.assign(wait, {
      cancel: () => {
        if (done) return
        done = true
        call(addon.readCancel, fence)
      }
    })
  }

  /** Gpu.read: readStart, awaited. */
  read (t, rect) { return this.readStart(t, rect)() }

  /** Gpu.readNow (gl.ts:658-700): blocking. */
  readNow (t, rect = { x: 0, y: 0, width: t.width, height: t.height }) {
    const texel = t.bytes / (t.width * t.height)
    const band = rect.height * t.width * texel
    const ab = call(addon.readNow, this.ctx, t.tex, rect.y * t.width * texel, band)
    return cut(ab, t, rect, texel)
  }

  /** Gpu.flush (gl.ts:729-732); PacedGpu.finish. */
  flush () { call(addon.flush, this.ctx) }
  finish () { call(addon.finish, this.ctx) }

  /** Gpu.dispose (gl.ts:316-331): every texture and the context. */
  dispose () {
    if (this.lost) return
    this.lost = true
    this.live.clear()
    call(addon.ctxDestroy, this.ctx)
  }

  /**
   * Native kernels over textures, one per family of the engine's passes. A
   * matrix is {N, K, layout, zero, quants, scales?, zeros?} with textures
   * holding the QuantMatrix arrays (src/weights.ts:1-31).
   */
  get ops () {
    const ctx = this.ctx
    const m = (w) => ({
      N: w.N,
      K: w.K,
      layout: w.layout,
      zero: w.zero,
      quants: w.quants.tex,
      scales: w.scales ? w.scales.tex : null,
      zeros: w.zeros ? w.zeros.tex : null
    })
    return {
      /** The loaders' packers on the GPU (packQ4_0, packQ4_K: src/repack.ts:60-168). */
      repack: (kind, w, row0, rows, src, srcRows) =>
        call(addon.repack, ctx, kind, m(w), row0, rows, src.tex, srcRows ? srcRows.tex : null),
      /** matrixRow (src/repack.ts:865-891) into an R32F texture. */
      dequant: (w, row0, rows, out) => call(addon.dequant, ctx, m(w), row0, rows, out.tex),
      /** splitPartials + pf (src/engine.ts:5241-5377): y = x W^T for M rows of halves. */
      gemv: (w, x, M, y) => call(addon.gemv, ctx, m(w), x.tex, M, y.tex),
      /** Engine.argmax (src/engine.ts:8271-8336): the first largest logit of each row. */
      argmax: (logits, M, V, ids, scratch) => call(addon.argmax, ctx, logits.tex, M, V, ids.tex, scratch.tex),
      argmaxScratchBytes: (M, V) => addon.argmaxScratchBytes(M, V)
    }
  }
}

/** The matrix arrays' sizes (src/weights.ts:153-178). */
function quantSizes (N, K, layout = addon.constants.LAYOUT_ROWGROUP, zero = addon.constants.ZERO_8) {
  return call(addon.q4Sizes, N, K, layout, zero)
}

module.exports = {
  HipGpu,
  GpuError,
  GL,
  TEXEL_BYTES,
  quantSizes,
  ggufHeader: (p) => call(addon.ggufHeader, p),
  onnxGraph: (p) => call(addon.onnxGraph, p),
  version: () => addon.version(),
  constants: addon.constants,
  addon
}
