"""The reference's weight-free decoder fixture, restated in Python (test
infrastructure).  It follows the reference's own CPU model of the fixture,
native/qwen3-tts-native-codec/src/reference.rs:3-70 (the same arithmetic the
CUDA fixture kernels run, native/qwen3-tts-native-codec/native/src/
codec_state.cu:185-318), and its frame generator and packet pattern,
native/qwen3-tts-native-codec/src/main.rs:1483-1500, 1944-1956.
"""
import numpy as np

STRIDES = (8, 5, 4, 3)


def _div4(x):
    """C / Rust integer division by 4 (truncates toward zero)."""
    return int(x / 4) if x >= 0 else -((-x) // 4)


def deterministic_frames(count):
    state = 0x6D2B79F5
    frames = np.zeros((count, 16), np.uint16)
    for f in range(count):
        for c in range(16):
            state = (state * 1_664_525 + 1_013_904_223) & 0xFFFFFFFF
            frames[f, c] = (state >> 8) & 2047
    return frames


class FixtureState:
    def __init__(self):
        self.preconv = [0, 0]
        self.tails = [[0] * s for s in STRIDES]

    def process(self, frames):
        values = []
        for frame in np.asarray(frames):
            weighted = sum(int(code & 2047) * (i + 1) for i, code in enumerate(frame))
            centered = (weighted & 4095) - 2048
            values.append(_div4(3 * centered + 2 * self.preconv[0] - self.preconv[1]))
            self.preconv = [centered, self.preconv[0]]
        values = [v for v in values for _ in range(4)]  # repeat x2, x2
        for stage, stride in enumerate(STRIDES):
            tail = self.tails[stage]
            out = []
            for i, v in enumerate(values):
                for phase in range(stride):
                    previous = tail[phase] if i == 0 else values[i - 1]
                    out.append(_div4(3 * v + previous))
            self.tails[stage] = [values[-1]] * stride
            values = out
        return np.clip(np.array(values, np.int64) * 8, -32768, 32767).astype(np.int16)


PACKET_PATTERN = (1, 4, 2, 3, 4, 1, 3, 2)


def packets(total):
    out, position, k = [], 0, 0
    while position < total:
        count = min(PACKET_PATTERN[k % len(PACKET_PATTERN)], total - position)
        out.append((position, position + count))
        position += count
        k += 1
    return out
