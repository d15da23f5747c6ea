// DecodeRunner: one global decode step over the shared KV ring and the 17-step
// local frame head, mirroring the reference's DecodeRunner
// (src/lib/tts/engine/decode.ts:201-1046): globalStep, nextFrame,
// nextFrameSteps, clearSeen, maxSlotCount, dispose.
import { AUDIO_PAD_ID, orDefault, ROW_WIDTH } from "./native.mjs";

export class DecodeRunner {
  /**
   * @param native   the addon
   * @param handle   the context shared with the PrefillRunner
   * @param maxSlots global KV ring slots
   * @param settings LocalHeadSettings {audioEndTokenId, audioAssistantSlotTokenId, repetitionPenalty}
   */
  constructor(native, handle, maxSlots, settings) {
    this.native = native;
    this.handle = handle;
    this.maxSlots = maxSlots;
    this.settings = settings;
    native.setLocalHead(
      handle,
      settings.audioEndTokenId,
      settings.audioAssistantSlotTokenId,
      settings.repetitionPenalty,
    );
    this.clearSeen();
  }

  /** Forget the repetition-penalty history: a new utterance starts clean (decode.ts:276-280). */
  clearSeen() {
    this.native.clearSeen(this.handle, null);
  }

  /**
   * One global step at `position`: embed the 17-wide row, run every layer
   * (appending this row's K/V) and return ln_f, [768] (decode.ts:712-775).
   * A position beyond a non-wrapping ring throws the reference's error.
   */
  async globalStep(row, position, _layers, _lnF, _embed) {
    const staged = new Int32Array(ROW_WIDTH);
    for (let i = 0; i < ROW_WIDTH; i += 1) staged[i] = orDefault(row[i], AUDIO_PAD_ID);
    return this.native.decodeStepAsync(this.handle, 1, staged, Int32Array.of(position));
  }

  /**
   * The local head: 17 sequential steps producing one frame of 16 codes, or
   * null when the text head chooses audio_end (decode.ts:788-939).
   */
  async nextFrame(hidden, _embed) {
    const r = await this.native.localFrameAsync(this.handle, 1, hidden);
    if (!r.cont[0]) return null;
    return Array.from(r.codes);
  }

  /** Run local-head steps 0 .. maxStep and return the last ln_f (decode.ts:970-1030). */
  async nextFrameSteps(hidden, _embed, maxStep) {
    return this.native.localSteps(this.handle, 1, hidden, maxStep);
  }

  /** number of slots in the global KV ring */
  get maxSlotCount() {
    return this.maxSlots;
  }

  dispose() {}
}
